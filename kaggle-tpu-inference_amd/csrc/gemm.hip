// Prefill GEMMs on MFMA (gfx950 v_mfma_f32_16x16x32_bf16).
//
// C[m, n] = sum_k A[m, k] * B[n, k]: activations A [M, K] and weights B [N, K]
// are both row-major with K contiguous, as every projection of the model is
// stored (model.py:84-117), so both operands stream 16-byte rows.  bf16 in,
// f32 accumulate.  One block computes a BM x BN tile with 4 waves (2 x 2);
// a wave holds (BM/2) x (BN/2) of f32 accumulators as 16 x 16 MFMA tiles.
// K advances 32 at a time through double-buffered LDS tiles: the next step's
// global loads are in flight while the current step multiplies.
//
// MFMA operand layout (16x16x32 bf16): lane l holds A[l%16][8(l/16)..+7] and
// B[l%16][8(l/16)..+7] (both rows of their K-contiguous tiles) and receives
// C[4(l/16)+i][l%16], i < 4.
//
// Options, used by the batched prefill:
//  * a_rows: A row of output row m is a_rows[m] (token gather for the MoE);
//  * grouped tiles: a device list of (group, m0, m1) M-tiles, each using the
//    group's B (b + group * b_group_stride) -- one expert per tile;
//  * split-K: blockIdx.z takes K slice z and writes f32 partials, summed in
//    slice order by gemm_reduce_kernel (deterministic);
//  * epilogues: bf16 store, f32 store, or the gated activation of a (gate, up)
//    pair: the tile's first BN/2 B rows come from b, the last BN/2 from
//    b + pair_offset at the same row index, and output column n0/2 + j gets
//    bf16(bf16(bf16(gelu(bf16(g))) * bf16(u)) * bf16(w_row)) (model.py:220,
//    model.py:246-247 and 269-271 with the routing weight w_row of the row).
#include <stdlib.h>

#include <type_traits>

#include "capi_util.h"
#include "common.h"

namespace g4mi {

enum { kEpBf16 = 0, kEpF32 = 1, kEpGated = 2 };

struct GemmTile {
  int32_t group, m0, m1;
};

constexpr int kMaxSeg = 4;

struct GemmArgs {
  const uint16_t* a;
  int64_t lda;
  const int32_t* a_rows;    // null: identity
  const uint16_t* b;
  int64_t ldb;
  int64_t b_group_stride;   // elements between groups (grouped tiles)
  int64_t pair_offset;      // gated: element offset of the up rows
  int M, N, K;              // N: output columns (gated: gate rows)
  const GemmTile* tiles;    // null: plain M tiling
  const int32_t* ntiles;    // device count of `tiles`
  void* c;
  int64_t ldc;
  const float* row_scale;   // gated: per output row weight (null: 1)
  int k_slices;             // split-K slices (f32 partials when > 1)
  float* partial;           // [k_slices, M, N] f32
  // column segments (skinny kernel only): nseg > 0 splits the N output
  // columns at seg_end[]; segment s reads its own B rows seg_b[s] and writes
  // its own C seg_c[s] (row stride = the segment's width)
  int nseg;
  int seg_end[kMaxSeg];
  const uint16_t* seg_b[kMaxSeg];
  void* seg_c[kMaxSeg];
};

constexpr int kBK = 64;  // K per pipeline step
constexpr int kPad = 8;  // LDS row padding (elements): rows of 144 bytes

template <int BM, int BN, int EP>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs g) {
  constexpr int WM = BM / 2, WN = BN / 2;   // wave tile
  constexpr int FM = WM / 16, FN = WN / 16; // MFMA fragments per wave
  constexpr int LDT = kBK + kPad;
  constexpr int CPR = kBK / 8;              // 16-byte chunks per tile row
  constexpr int ACH = BM * CPR / 256;       // A chunks per thread per step
  constexpr int BCH = BN * CPR / 256;
  static_assert(ACH >= 1 && BCH >= 1, "tile too small for 256 threads");
  // one LDS block: the double-buffered A and B tiles, reused by the gated
  // epilogue's exchange
  __shared__ __align__(16) uint16_t smem[2 * BM * LDT + 2 * BN * LDT];
  // A tile of buffer `buf` at smem + buf*BM*LDT, B tile at smem + 2*BM*LDT + buf*BN*LDT
  constexpr int SB0 = 2 * BM * LDT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- this block's tile
  int group = 0, m0, m1;
  if (g.tiles != nullptr) {
    if ((int)blockIdx.x >= g.ntiles[0]) return;
    const GemmTile t = g.tiles[blockIdx.x];
    group = t.group;
    m0 = t.m0;
    m1 = t.m1;
  } else {
    m0 = blockIdx.x * BM;
    m1 = min(g.M, m0 + BM);
  }
  const int n0 = blockIdx.y * (EP == kEpGated ? BN / 2 : BN);  // first output column
  const uint16_t* bbase = g.b + (size_t)group * g.b_group_stride;
  const int kslices = g.k_slices;
  const int ksteps_all = g.K / kBK;
  const int ks0 = (ksteps_all * (int)blockIdx.z) / kslices;
  const int ks1 = (ksteps_all * ((int)blockIdx.z + 1)) / kslices;

  // ---- global source rows of the chunks this thread copies (fixed over K)
  const u32x4* asrc[ACH];
  const u32x4* bsrc[BCH];
  int adst[ACH], bdst[BCH];
#pragma unroll
  for (int q = 0; q < ACH; ++q) {
    const int c = tid + 256 * q;  // chunk: row c/CPR, 8 elements at (c%CPR)*8
    const int r = c / CPR, kc = (c % CPR) * 8;
    const int m = min(m0 + r, max(m1 - 1, m0));
    const int src = (g.a_rows != nullptr) ? g.a_rows[m] : m;
    asrc[q] = (const u32x4*)(g.a + (size_t)src * g.lda + kc);
    adst[q] = r * LDT + kc;
  }
#pragma unroll
  for (int q = 0; q < BCH; ++q) {
    const int c = tid + 256 * q;
    const int r = c / CPR, kc = (c % CPR) * 8;
    const uint16_t* row;
    if constexpr (EP == kEpGated) {
      const int half = r >= BN / 2;
      const int n = min(n0 + (r - half * (BN / 2)), g.N - 1);
      row = bbase + (half ? g.pair_offset : 0) + (size_t)n * g.ldb;
    } else {
      const int n = min(n0 + r, g.N - 1);
      row = bbase + (size_t)n * g.ldb;
    }
    bsrc[q] = (const u32x4*)(row + kc);
    bdst[q] = r * LDT + kc;
  }

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Pipeline: tile j's global loads go to register stage j%2 two steps
  // before it is multiplied; at step k the block multiplies LDS buffer k%2,
  // stores register stage (k+1)%2 (tile k+1) into the other buffer and has
  // tile k+2's loads in flight, so two steps of MFMA work cover each load.
  u32x4 ra[2][ACH], rb[2][BCH];
  auto gload = [&](int ks, u32x4* a_, u32x4* b_) {
#pragma unroll
    for (int q = 0; q < ACH; ++q) a_[q] = ld16(asrc[q] + ks * CPR);
#pragma unroll
    for (int q = 0; q < BCH; ++q) b_[q] = ld_stream(bsrc[q] + ks * CPR);
  };
  auto lstore = [&](int buf, const u32x4* a_, const u32x4* b_) {
#pragma unroll
    for (int q = 0; q < ACH; ++q) *(u32x4*)(smem + buf * BM * LDT + adst[q]) = a_[q];
#pragma unroll
    for (int q = 0; q < BCH; ++q) *(u32x4*)(smem + SB0 + buf * BN * LDT + bdst[q]) = b_[q];
  };
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      u32x4 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *(const u32x4*)(smem + buf * BM * LDT + (wm * WM + i * 16 + fr) * LDT + 32 * kk + fk);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *(const u32x4*)(smem + SB0 + buf * BN * LDT + (wn * WN + j * 16 + fr) * LDT + 32 * kk + fk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[i]),
                                                              __builtin_bit_cast(bf16x8, bf[j]), acc[i][j], 0, 0,
                                                              0);
    }
  };
  // one pipeline step on buffer BUF (register stages are compile-time)
  auto step = [&](int ks, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    if (ks + 2 < ks1) gload(ks + 2, ra[BUF], rb[BUF]);
    compute(BUF);
    if (ks + 1 < ks1) lstore(BUF ^ 1, ra[BUF ^ 1], rb[BUF ^ 1]);
    __syncthreads();
  };
  if (ks0 < ks1) {
    gload(ks0, ra[0], rb[0]);
    if (ks0 + 1 < ks1) gload(ks0 + 1, ra[1], rb[1]);
    lstore(0, ra[0], rb[0]);
    __syncthreads();
    int ks = ks0;
    for (; ks + 1 < ks1; ks += 2) {
      step(ks, std::integral_constant<int, 0>{});
      step(ks + 1, std::integral_constant<int, 1>{});
    }
    if (ks < ks1) step(ks, std::integral_constant<int, 0>{});
  }

  // ---- epilogue.  Fragment (i, j), register q: row wm*WM + 16i + 4(l/16) + q,
  // column wn*WN + 16j + (l%16) of the tile.
  const int er = 4 * (lane >> 4), ec = lane & 15;
  if (kslices > 1) {
    float* p = g.partial + (size_t)blockIdx.z * g.M * g.N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int m = m0 + wm * WM + 16 * i + er + q, n = n0 + wn * WN + 16 * j + ec;
          if (m < m1 && n < g.N) p[(size_t)m * g.N + n] = acc[i][j][q];
        }
    return;
  }
  if constexpr (EP == kEpGated) {
    // up (wn = 1) to LDS, then the gate waves combine
    __syncthreads();
    float* su = (float*)smem;  // BM x WN f32
    static_assert((size_t)BM * (BN / 2) * 4 <= sizeof(smem), "exchange buffer too small");
    if (wn == 1) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) su[(wm * WM + 16 * i + er + q) * WN + 16 * j + ec] = acc[i][j][q];
    }
    __syncthreads();
    if (wn == 0) {
      uint16_t* c = (uint16_t*)g.c;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r = wm * WM + 16 * i + er + q, col = 16 * j + ec;
            const int m = m0 + r, n = n0 + col;
            if (m < m1 && n < g.N) {
              const float gt = rbf(acc[i][j][q]), up = rbf(su[r * WN + col]);
              float a = rbf(rbf(gelu_tanh(gt)) * up);
              if (g.row_scale != nullptr) a = rbf(a * rbf(g.row_scale[m]));
              c[(size_t)m * g.ldc + n] = f2bf(a);
            }
          }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + wm * WM + 16 * i + er + q, n = n0 + wn * WN + 16 * j + ec;
        if (m < m1 && n < g.N) {
          if constexpr (EP == kEpF32) ((float*)g.c)[(size_t)m * g.ldc + n] = acc[i][j][q];
          else ((uint16_t*)g.c)[(size_t)m * g.ldc + n] = f2bf(acc[i][j][q]);
        }
      }
}

// ---- skinny GEMM (M <= 16 rows: batched decode, short prompts)
// A block owns 16*NTL output columns (B rows; with the gated epilogue the
// gate and the up rows) for all M <= 16 A rows; its 4 waves split K into
// quarters.  Per k-step a wave loads one A fragment and multiplies it into
// NTL 16x16 MFMA chains (A rows beyond M are clamped duplicates and are not
// stored).  The wave partials meet in LDS and are summed in wave order, so
// there is no split-K reduce kernel.  Each wave requests CHK k-steps of A and
// B -- its whole K quarter when that fits, so one round trip -- before the
// first multiply.  NTL = 4 amortises the A fragments over 64 columns when N
// is large (the lm_head); NTL = 1 keeps ceil(N/16) blocks for the layer
// projections.  With column segments (NTL = 1) a block's 16 columns lie in
// one segment, whose B rows and C it uses.
template <int EP, int NTL, int CHK, int NWV = 4>
__global__ __launch_bounds__(64 * NWV) void gemm_skinny_kernel(GemmArgs g) {
  constexpr bool GATED = EP == kEpGated;
  constexpr int NP = GATED ? 2 : 1;         // B row sets (gate, up)
  __shared__ float part[NP][NWV][16][16 * NTL + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  int n0 = blockIdx.x * 16 * NTL;
  const uint16_t* bmat = g.b;
  void* cmat = g.c;
  int ncols = g.N;
  int64_t ldb = g.ldb, ldc = g.ldc;
  if (g.nseg > 0) {  // block-uniform: selects, no indexed kernel arguments
    int sg = 0;
#pragma unroll
    for (int i = 0; i + 1 < kMaxSeg; ++i) sg += (i + 1 < g.nseg && n0 >= g.seg_end[i]) ? 1 : 0;
    const int lo = (sg == 0) ? 0 : (sg == 1) ? g.seg_end[0] : (sg == 2) ? g.seg_end[1] : g.seg_end[2];
    const int hi = (sg == 0) ? g.seg_end[0] : (sg == 1) ? g.seg_end[1] : (sg == 2) ? g.seg_end[2] : g.seg_end[3];
    bmat = (sg == 0) ? g.seg_b[0] : (sg == 1) ? g.seg_b[1] : (sg == 2) ? g.seg_b[2] : g.seg_b[3];
    cmat = (sg == 0) ? g.seg_c[0] : (sg == 1) ? g.seg_c[1] : (sg == 2) ? g.seg_c[2] : g.seg_c[3];
    n0 -= lo;
    ncols = hi - lo;
    ldb = g.K;
    ldc = ncols;
  }
  const int ksteps = g.K / 32;
  const int s0 = (ksteps * wave) / NWV, s1 = (ksteps * (wave + 1)) / NWV;
  const int m = min(fr, g.M - 1);
  const int arow = (g.a_rows != nullptr) ? g.a_rows[m] : m;
  const u32x4* ap = (const u32x4*)(g.a + (size_t)arow * g.lda + fk);
  const u32x4* bp[NP][NTL];
#pragma unroll
  for (int t = 0; t < NTL; ++t) {
    const int n = min(n0 + 16 * t + fr, ncols - 1);
    bp[0][t] = (const u32x4*)(bmat + (size_t)n * ldb + fk);
    if constexpr (GATED) bp[NP - 1][t] = (const u32x4*)(bmat + g.pair_offset + (size_t)n * ldb + fk);
  }
  f32x4 acc[NP][NTL];
#pragma unroll
  for (int q = 0; q < NP; ++q)
#pragma unroll
    for (int t = 0; t < NTL; ++t) acc[q][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = s0; c0 < s1; c0 += CHK) {
    u32x4 af[CHK], bf[NP][NTL][CHK];
#pragma unroll
    for (int j = 0; j < CHK; ++j) {
      const int st = min(c0 + j, s1 - 1);  // clamped: always in range
      af[j] = ld16(ap + st * 4);
#pragma unroll
      for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int t = 0; t < NTL; ++t) bf[q][t][j] = ld16(bp[q][t] + st * 4);
    }
    // every load of the chunk is issued before the first wait
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < CHK; ++j) {
      // a clamped step past the wave's range multiplies a zero A fragment
      // (a select, not a branch: the loads stay where they were issued)
      const u32x4 aj = (c0 + j < s1) ? af[j] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int t = 0; t < NTL; ++t)
          acc[q][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, aj),
                                                              __builtin_bit_cast(bf16x8, bf[q][t][j]), acc[q][t], 0, 0,
                                                              0);
    }
  }
  // C layout: row (A row) 4*(l/16)+i, column (output n) 16*t + l%16
#pragma unroll
  for (int q = 0; q < NP; ++q)
#pragma unroll
    for (int t = 0; t < NTL; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[q][wave][4 * (lane >> 4) + i][16 * t + fr] = acc[q][t][i];
  __syncthreads();
  for (int e = tid; e < 16 * 16 * NTL; e += 64 * NWV) {  // one output per (row, column)
    const int r = e / (16 * NTL), c = e % (16 * NTL);
    const int mo = r, no = n0 + c;
    if (mo >= g.M || no >= ncols) continue;
    float v = part[0][0][r][c];
#pragma unroll
    for (int w = 1; w < NWV; ++w) v += part[0][w][r][c];
    if constexpr (GATED) {
      float uv = part[1][0][r][c];
#pragma unroll
      for (int w = 1; w < NWV; ++w) uv += part[1][w][r][c];
      float act = rbf(rbf(gelu_tanh(rbf(v))) * rbf(uv));
      if (g.row_scale != nullptr) act = rbf(act * rbf(g.row_scale[mo]));
      ((uint16_t*)cmat)[(size_t)mo * ldc + no] = f2bf(act);
    } else if constexpr (EP == kEpF32) {
      ((float*)cmat)[(size_t)mo * ldc + no] = v;
    } else {
      ((uint16_t*)cmat)[(size_t)mo * ldc + no] = f2bf(v);
    }
  }
}

// C = sum over the k_slices f32 partials, in slice order.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float* __restrict__ partial, int slices, int64_t mn,
                                                          int N, void* c, int64_t ldc, int f32_out) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= mn) return;
  float s = 0.0f;
  for (int z = 0; z < slices; ++z) s += partial[(size_t)z * mn + e];
  const int64_t m = e / N, n = e - m * N;
  if (f32_out) ((float*)c)[m * ldc + n] = s;
  else ((uint16_t*)c)[m * ldc + n] = f2bf(s);
}

template <int BM, int BN, int EP>
static void launch(const GemmArgs& g, int mtiles, hipStream_t st) {
  const int ncols = (EP == kEpGated) ? BN / 2 : BN;
  dim3 grid((unsigned)mtiles, (unsigned)((g.N + ncols - 1) / ncols), (unsigned)g.k_slices);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, EP>), grid, dim3(256), 0, st, g);
}

}  // namespace g4mi

using namespace g4mi;

extern "C" {

int64_t g4mi_gemm_workspace_bytes(int64_t M, int64_t N, int64_t k_slices) {
  return k_slices > 1 ? k_slices * M * N * 4 : 0;
}

int g4mi_gemm_bf16(const uint16_t* a, int64_t lda, const int32_t* a_rows, const uint16_t* b, int64_t ldb,
                   int64_t b_group_stride, int64_t pair_offset, int64_t M, int64_t N, int64_t K,
                   const int32_t* tiles, const int32_t* ntiles, int64_t max_tiles, int32_t epilogue, void* c,
                   int64_t ldc, const float* row_scale, int64_t k_slices, void* ws, int64_t ws_bytes,
                   void* stream) {
  G4MI_REQUIRE(a && b && c && M >= 1 && N >= 1 && K >= 1, G4MI_EINVAL, "gemm: missing argument");
  G4MI_REQUIRE(K % kBK == 0, G4MI_EUNSUPPORTED, "gemm: K=%lld must be a multiple of %d", (long long)K, kBK);
  G4MI_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && ((uintptr_t)a & 15u) == 0 && ((uintptr_t)b & 15u) == 0, G4MI_EALIGN,
               "gemm: operand rows must be 16-byte aligned");
  G4MI_REQUIRE(epilogue >= kEpBf16 && epilogue <= kEpGated, G4MI_EINVAL, "gemm: bad epilogue %d", epilogue);
  G4MI_REQUIRE(epilogue != kEpGated || (pair_offset % 8 == 0 && pair_offset != 0), G4MI_EINVAL,
               "gemm: the gated epilogue needs the up rows' offset");
  G4MI_REQUIRE(tiles == nullptr || (ntiles && max_tiles >= 1), G4MI_EINVAL, "gemm: grouped tiles need a count");
  G4MI_REQUIRE(k_slices >= 1 && k_slices <= K / kBK && k_slices <= 64, G4MI_EINVAL, "gemm: bad k_slices");
  G4MI_REQUIRE(k_slices == 1 || (tiles == nullptr && epilogue != kEpGated), G4MI_EUNSUPPORTED,
               "gemm: split-K is for plain bf16/f32 outputs");
  G4MI_REQUIRE(k_slices == 1 || (ws && ws_bytes >= g4mi_gemm_workspace_bytes(M, N, k_slices)), G4MI_EWORKSPACE,
               "gemm: workspace too small for split-K");
  GemmArgs g;
  g.a = a; g.lda = lda; g.a_rows = a_rows; g.b = b; g.ldb = ldb; g.b_group_stride = b_group_stride;
  g.pair_offset = pair_offset; g.M = (int)M; g.N = (int)N; g.K = (int)K; g.tiles = (const GemmTile*)tiles;
  g.ntiles = ntiles; g.c = c; g.ldc = ldc; g.row_scale = row_scale; g.k_slices = (int)k_slices;
  g.partial = (float*)ws;
  g.nseg = 0;
  hipStream_t st = as_stream(stream);
  if (tiles == nullptr && M <= 16 && k_slices == 1) {
    if (N >= 16384 && epilogue != kEpGated) {  // wide: 64 columns per block
      const dim3 grid((unsigned)((N + 63) / 64));
      if (epilogue == kEpF32) hipLaunchKernelGGL((gemm_skinny_kernel<kEpF32, 4, 8>), grid, dim3(256), 0, st, g);
      else hipLaunchKernelGGL((gemm_skinny_kernel<kEpBf16, 4, 8>), grid, dim3(256), 0, st, g);
    } else {
      // a wave's whole K quarter in one request when it is at most 24 (or 32) steps
      const dim3 grid((unsigned)((N + 15) / 16));
      const bool wide = (K / 32 + 3) / 4 > 24;
#define G4MI_SKINNY(E)                                                                          \
  if (wide) hipLaunchKernelGGL((gemm_skinny_kernel<E, 1, 32>), grid, dim3(256), 0, st, g);      \
  else hipLaunchKernelGGL((gemm_skinny_kernel<E, 1, 24>), grid, dim3(256), 0, st, g);
      if (epilogue == kEpGated) { G4MI_SKINNY(kEpGated) }
      else if (epilogue == kEpF32) { G4MI_SKINNY(kEpF32) }
      else { G4MI_SKINNY(kEpBf16) }
#undef G4MI_SKINNY
    }
    return check_launch("gemm_bf16 (skinny)");
  }
  // grouped tiles are up to 128 rows (128-row kernels); small plain M takes 64-row tiles
  const bool small = tiles == nullptr && M <= 64;
  const int64_t mtiles = tiles ? max_tiles : (M + (small ? 63 : 127)) / (small ? 64 : 128);
  G4MI_REQUIRE(mtiles <= 2147483647, G4MI_EINVAL, "gemm: too many tiles");
  if (small) {
    if (epilogue == kEpGated) launch<64, 128, kEpGated>(g, (int)mtiles, st);
    else if (k_slices > 1 || epilogue == kEpF32) launch<64, 64, kEpF32>(g, (int)mtiles, st);
    else launch<64, 64, kEpBf16>(g, (int)mtiles, st);
  } else {
    if (epilogue == kEpGated) launch<128, 128, kEpGated>(g, (int)mtiles, st);
    else if (k_slices > 1 || epilogue == kEpF32) launch<128, 128, kEpF32>(g, (int)mtiles, st);
    else launch<128, 128, kEpBf16>(g, (int)mtiles, st);
  }
  if (k_slices > 1) {
    const int64_t mn = M * N;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st, (const float*)ws,
                       (int)k_slices, mn, (int)N, c, ldc, epilogue == kEpF32 ? 1 : 0);
  }
  return check_launch("gemm_bf16");
}

int g4mi_gemm_bf16_segments(const uint16_t* a, int64_t lda, int64_t M, int64_t K, int32_t nseg,
                            const uint16_t* const* b, const int64_t* n, uint16_t* const* c, void* stream) {
  G4MI_REQUIRE(a && b && n && c && nseg >= 1 && nseg <= kMaxSeg, G4MI_EINVAL,
               "gemm_segments: need 1..%d segments", kMaxSeg);
  G4MI_REQUIRE(M >= 1 && M <= 16, G4MI_EUNSUPPORTED, "gemm_segments: M=%lld not in [1, 16]", (long long)M);
  G4MI_REQUIRE(K >= kBK && K % kBK == 0, G4MI_EUNSUPPORTED, "gemm_segments: K=%lld must be a multiple of %d",
               (long long)K, kBK);
  G4MI_REQUIRE(lda % 8 == 0 && ((uintptr_t)a & 15u) == 0, G4MI_EALIGN, "gemm_segments: A rows must be 16-byte aligned");
  GemmArgs g = {};
  g.a = a; g.lda = lda; g.M = (int)M; g.K = (int)K; g.ldb = K; g.k_slices = 1; g.nseg = nseg;
  int64_t end = 0;
  for (int s = 0; s < kMaxSeg; ++s) {
    if (s < nseg) {
      G4MI_REQUIRE(b[s] && c[s] && ((uintptr_t)b[s] & 15u) == 0, G4MI_EALIGN,
                   "gemm_segments: segment %d needs 16-byte aligned B rows and a C", s);
      G4MI_REQUIRE(n[s] >= 16 && n[s] % 16 == 0, G4MI_EUNSUPPORTED,
                   "gemm_segments: segment %d width %lld must be a positive multiple of 16", s, (long long)n[s]);
      end += n[s];
      G4MI_REQUIRE(end <= 2147483647, G4MI_EINVAL, "gemm_segments: too many columns");
      g.seg_b[s] = b[s]; g.seg_c[s] = c[s];
    } else {
      g.seg_b[s] = b[nseg - 1]; g.seg_c[s] = c[nseg - 1];
    }
    g.seg_end[s] = (int)end;
  }
  g.b = g.seg_b[0]; g.c = g.seg_c[0]; g.N = (int)end; g.ldc = n[0];
  const dim3 grid((unsigned)(end / 16));
  hipStream_t st = as_stream(stream);
  if ((K / 32 + 3) / 4 > 24) hipLaunchKernelGGL((gemm_skinny_kernel<kEpBf16, 1, 32>), grid, dim3(256), 0, st, g);
  else hipLaunchKernelGGL((gemm_skinny_kernel<kEpBf16, 1, 24>), grid, dim3(256), 0, st, g);
  return check_launch("gemm_bf16_segments");
}

}  // extern "C"
