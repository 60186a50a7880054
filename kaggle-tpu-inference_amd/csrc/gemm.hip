// Prefill GEMMs on MFMA (gfx950 v_mfma_f32_16x16x32_bf16).
//
// C[m, n] = sum_k A[m, k] * B[n, k]: activations A [M, K] and weights B [N, K]
// are both row-major with K contiguous, as every projection of the model is
// stored (model.py:84-117), so both operands stream 16-byte rows.  bf16 in,
// f32 accumulate.  More than 16 rows: a tile kernel (4 waves, 128 x 128 or
// 64 x 128 tiles) fed by direct global->LDS loads through 2 or 3 LDS stages
// (see gemm_kernel); up to 16 rows: a skinny kernel that splits K over the
// waves of a block (gemm_skinny_kernel).
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
//    pair: the tile's first BN/2 B rows are gate rows n0 + j of b, the last
//    BN/2 the up rows at b + pair_offset, and output column n0 + j gets
//    bf16(bf16(bf16(gelu(bf16(g))) * bf16(u)) * bf16(w_row)) (model.py:220,
//    model.py:246-247 and 269-271 with the routing weight w_row of the row).
#include <stdlib.h>

#include <type_traits>
#include <utility>

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

constexpr int kBK = 64;  // K per pipeline stage

// Waves per block of the 16-column skinny products (gemm_skinny_kernel with
// NTL = 1): 8 by default, so that each wave's eighth of K (up to 12 or 16
// steps of A and B) is one request that fits its registers; with 4 waves a
// quarter of the 2,816-wide gated product (22 steps of A, gate and up) needs
// more than 256 VGPRs and the compiler splits the request.  At 8 rows the
// batched decode step 6.40 -> 6.34 ms.  G4MI_SKINNY_WAVES=4 keeps 4 waves.
static bool skinny_8_waves() {
  const char* e = getenv("G4MI_SKINNY_WAVES");
  return e == nullptr || atoi(e) != 4;
}

// ---- tile GEMM (M > 16 rows)
// A block computes a BM x BN tile (BM, BN in {64, 128, ...}) with 4 waves
// (2 x 2), each a (BM/2) x (BN/2) patch of 16 x 16 MFMA accumulators.  K
// advances kBK = 64 per stage through ST LDS stages (separate __shared__
// arrays), filled by direct global->LDS loads (global_load_lds_dwordx4: 64
// lanes x 16 bytes = 1 KB per instruction, written contiguously in lane
// order).  Each tile row is 8 slots of 16 bytes; slot (r, p) holds k-chunk
// p ^ sw(r), sw(r) = (r & 7) ^ ((r >> 3) & 1), so the fragment reads (16
// rows x one chunk per ds_read_b128) hit distinct banks for 8 or 16 lanes
// per cycle.  Stage step ks:
//   phase A: the MFMAs of k-half 0 with the reads of k-half 1 in between;
//   wait for those reads and for step ks+1's DMA, barrier (step ks+1's stage
//   landed in every wave; stage ks read by every wave);
//   phase B: the MFMAs of k-half 1 with the reads of step ks+1's k-half 0
//   and the DMA of step ks+ST (into stage ks % ST) in between.
// The DMA is inline asm (M0 = LDS address): the compiler sees no LDS
// writer, so it does not wait for every outstanding DMA before its own LDS
// reads (which it would for the builtin); the fragment reads are ordinary
// LDS loads whose waits and registers the compiler tracks, and the DMA waits
// are explicit (wait_vm_barrier).  sched_barrier pins the interleave; every
// loop over fragments is a static_for and every lambda always_inline, so
// the accumulators and fragments stay in registers.  ST = 2 stages let two
// blocks share a CU (OCC = 2), so one block's barrier overlaps the other's
// MFMAs; ST = 3 (one block per CU) covers more latency when there are fewer
// tiles than CUs.

// Waits until at most N of this wave's vector memory operations (the DMA of
// later steps) are outstanding and its LDS reads are done, then the barrier.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Tile of block `bid` of a 1-D grid: consecutive ids go to the 8 XCDs in
// turn (each XCD has its own L2), so XCD x takes the x-th contiguous run of
// the tile order.  Plain tiling: groups of 8 row tiles, column tiles inner
// (a group's A and B tiles are shared in the XCD's L2).  Grouped tiles
// (tile list order, column tiles inner): a run covers whole tiles, so an A
// tile is read once per XCD and the tiles of one group are neighbours.
// The grid holds 8 * ceil(max tiles / 8) blocks; with mtiles the live count
// (at most the maximum) block bid maps to id = (bid % 8) * per + bid / 8,
// one-to-one onto [0, nb) over the blocks with bid / 8 < per.  Returns false
// for every other block.
__host__ __device__ __forceinline__ bool tile_of(int bid, int mtiles, int ntiles_col, int& tx, int& ty,
                                                 bool grouped) {
  const int nb = mtiles * ntiles_col;
  const int per = (nb + 7) / 8;
  if (bid / 8 >= per) return false;
  const int id = (bid % 8) * per + bid / 8;
  if (id >= nb) return false;
  if (grouped) {
    tx = id / ntiles_col;
    ty = id % ntiles_col;
  } else {
    constexpr int G = 8;
    const int grp = id / (G * ntiles_col), fx = grp * G, gs = mtiles - fx < G ? mtiles - fx : G;
    tx = fx + (id % (G * ntiles_col)) % gs;
    ty = (id % (G * ntiles_col)) / gs;
  }
  return true;
}

// K-step offset per group of grouped tiles (coprime with the K step counts
// of the expert products, 44 and 11)
constexpr int kKRot = 7;

template <int BM, int BN, int ST, int OCC, int EP, bool GR>
__global__ __launch_bounds__(256, OCC) void gemm_kernel(GemmArgs g) {
  constexpr int WM = BM / 2, WN = BN / 2;    // wave tile
  constexpr int FM = WM / 16, FN = WN / 16;  // MFMA fragments per wave
  constexpr int AI = BM / 32, BI = BN / 32;  // DMA instructions per wave per stage
  constexpr int NL = AI + BI;
  constexpr int SB = (BM + BN) * 128;        // stage bytes
  constexpr int NF = FM + FN, NM = FM * FN;
  static_assert(ST == 2 || ST == 3, "2 or 3 stages");
  static_assert(AI >= 1 && BI >= 1, "tile too small for 256 threads");
  // the ST stages back to back in one array (two blocks of 80 KB, the
  // 192-row tiles, then fill the CU's 160 KB exactly)
  __shared__ __align__(1024) uint8_t stages[ST * SB];
  uint8_t* const st0 = stages;
  uint8_t* const st1 = stages + SB;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  constexpr int NCOL = (EP == kEpGated) ? BN / 2 : BN;  // output columns per tile
  const int ncol_tiles = (g.N + NCOL - 1) / NCOL;

  // ---- this block's tile
  int group = 0, m0, m1, tx, ty;
  if constexpr (GR) {  // grouped tiles (g.tiles)
    if (!tile_of(blockIdx.x, g.ntiles[0], ncol_tiles, tx, ty, true)) return;
    const GemmTile t = g.tiles[tx];
    group = t.group;
    m0 = t.m0;
    m1 = t.m1;
  } else {
    if (!tile_of(blockIdx.x, (g.M + BM - 1) / BM, ncol_tiles, tx, ty, false)) return;
    m0 = tx * BM;
    m1 = min(g.M, m0 + BM);
  }
  const int n0 = ty * NCOL;  // first output column
  const char* abase = (const char*)g.a;
  const char* bbase = (const char*)(g.b + (size_t)group * g.b_group_stride);
  const int kslices = g.k_slices;
  const int ksteps_all = g.K / kBK;
  const int ks0 = (ksteps_all * (int)blockIdx.z) / kslices;
  const int ks1 = (ksteps_all * ((int)blockIdx.z + 1)) / kslices;
  const int nks = ks1 - ks0;
  // grouped tiles start their K walk at an offset set by the group (the
  // tiles in flight then request different K slices of their weight rows),
  // and request their weights with the non-temporal policy (each weight byte
  // of a grouped product is read by one tile; the dense products' weights
  // are shared by every row tile and stay cached)
  const int krot = GR ? (group * kKRot) % ksteps_all : 0;

  // ---- DMA sources: instruction j of this wave fills tile rows
  // (wave*AI + j)*8 + lane/8, slot lane%8 (chunk (lane%8) ^ sw(row)).  Rows
  // past the tile repeat its last row (not stored).
  const char* asrc[AI];
  const char* bsrc[BI];
#pragma unroll
  for (int j = 0; j < AI; ++j) {
    const int r = (wave * AI + j) * 8 + (lane >> 3);
    const int cc = (lane & 7) ^ ((r & 7) ^ ((r >> 3) & 1));
    const int m = min(m0 + r, max(m1 - 1, m0));
    const int src = (g.a_rows != nullptr) ? g.a_rows[m] : m;
    asrc[j] = abase + ((int64_t)src * g.lda + cc * 8) * 2;
  }
#pragma unroll
  for (int j = 0; j < BI; ++j) {
    const int r = (wave * BI + j) * 8 + (lane >> 3);
    const int cc = (lane & 7) ^ ((r & 7) ^ ((r >> 3) & 1));
    int64_t row;
    if constexpr (EP == kEpGated) {
      const int half = r >= BN / 2;
      row = (half ? g.pair_offset : 0) + (int64_t)min(n0 + (r - half * (BN / 2)), g.N - 1) * g.ldb;
    } else {
      row = (int64_t)min(n0 + r, g.N - 1) * g.ldb;
    }
    bsrc[j] = bbase + (row + cc * 8) * 2;
  }
  // fragment reads: lane l takes row (l%16) of a 16-row block, chunk
  // 4*half + l/16 of the stage's 8 (byte offsets within a stage)
  const int swl = (lane & 7) ^ ((lane >> 3) & 1);
  uint32_t fa[2], fb[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int cch = (4 * kk + (lane >> 4)) ^ swl;
    fa[kk] = (uint32_t)(((wm * WM + (lane & 15)) * 8 + cch) * 16);
    fb[kk] = (uint32_t)(BM * 128 + ((wn * WN + (lane & 15)) * 8 + cch) * 16);
  }

  f32x4 acc[FM][FN];
  static_for<NM>([&](auto ic) __attribute__((always_inline)) { acc[decltype(ic)::value / FN][decltype(ic)::value % FN] = f32x4{0.0f, 0.0f, 0.0f, 0.0f}; });

  auto sbase = [&](auto sc) __attribute__((always_inline)) -> uint8_t* {
    constexpr int S = decltype(sc)::value;
    return stages + S * SB;
  };
  // DMA instruction q (< NL) of step ks into stage sc: 64 lanes x 16 bytes
  // from their global addresses to LDS[l, l + 1024) in lane order (M0 = l).
  // Inline asm: it has no register result, and the compiler, which does not
  // see an LDS writer, does not wait for it before its own LDS reads; the
  // waits are the explicit vmcnt waits below.
  auto issue1 = [&](int ks, auto sc, auto qc) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    uint8_t* s = sbase(sc);
    int kse = ks;
    if constexpr (GR) kse += krot - ((ks + krot >= ksteps_all) ? ksteps_all : 0);
    const uint32_t kb = (uint32_t)kse * kBK * 2u;
    const char* gp;
    uint32_t l;
    if constexpr (q < AI) {
      gp = asrc[q] + kb;
      l = (uint32_t)(uintptr_t)(s + (wave * AI + q) * 1024);
    } else {
      gp = bsrc[q - AI] + kb;
      l = (uint32_t)(uintptr_t)(s + BM * 128 + (wave * BI + q - AI) * 1024);
    }
    if constexpr (q >= AI && GR)
      asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                   :
                   : "v"(gp), "s"(__builtin_amdgcn_readfirstlane(l))
                   : "memory", "m0");
    else
      asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                   :
                   : "v"(gp), "s"(__builtin_amdgcn_readfirstlane(l))
                   : "memory", "m0");
  };
  struct Frag {
    u32x4 a[FM], b[FN];
  };
  // fragment read q (< NF) of k-half kk of stage sc (an ordinary LDS load:
  // the compiler waits for it before the MFMA that uses it)
  auto read1 = [&](Frag& f, auto sc, int kk, auto qc) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    const uint8_t* s = sbase(sc);
    if constexpr (q < FM) f.a[q] = *(const u32x4*)(s + fa[kk] + q * 16 * 128);
    else f.b[q - FM] = *(const u32x4*)(s + fb[kk] + (q - FM) * 16 * 128);
  };
  // 16-row fragments of this wave that hold rows of the tile (a grouped
  // tile may be short): the MFMAs of the others are skipped (wave-uniform)
  const int vfrag = min(FM, max(0, (m1 - (m0 + wm * WM) + 15) / 16));
  auto mfma1 = [&](const Frag& f, auto ic) __attribute__((always_inline)) {
    constexpr int i = decltype(ic)::value / FN, j = decltype(ic)::value % FN;
    if (i == 0 || i < vfrag)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, f.a[i]),
                                                          __builtin_bit_cast(bf16x8, f.b[j]), acc[i][j], 0, 0, 0);
  };
  using I = std::integral_constant<int, 0>;
  Frag f0, f1;
  // step t (relative to ks0) on stage S = t % ST; f0 holds its k-half 0
  // fragments (requested).  STD: not one of the last steps (every check true).
  auto step = [&](int t, auto sc, auto steady) __attribute__((always_inline)) {
    constexpr int S = decltype(sc)::value;
    constexpr bool STD = decltype(steady)::value;
    using SN = std::integral_constant<int, (S + 1) % ST>;
    static_for<NM>([&](auto ic) __attribute__((always_inline)) {
      constexpr int idx = decltype(ic)::value;
      mfma1(f0, ic);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (idx % 2 == 0 && idx / 2 < NF) read1(f1, sc, 1, std::integral_constant<int, idx / 2>{});
      __builtin_amdgcn_sched_barrier(0);
    });
    static_for<NF>([&](auto qc) __attribute__((always_inline)) {  // reads beyond the interleave slots
      if constexpr (decltype(qc)::value >= NM / 2) read1(f1, sc, 1, qc);
    });
    // this wave's LDS reads done; DMA still allowed in flight: steps t+2 ..
    // t+ST-1 (those that exist)
    if constexpr (STD) {
      wait_vm_barrier<(ST - 2) * NL>();
    } else {
      if (ST == 3 && t + 2 < nks) wait_vm_barrier<NL>();
      else wait_vm_barrier<0>();
    }
    const bool nxt = STD || t + 1 < nks, dma = STD || t + ST < nks;
    static_for<NM>([&](auto ic) __attribute__((always_inline)) {
      constexpr int idx = decltype(ic)::value;
      mfma1(f1, ic);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (idx % 2 == 0 && idx / 2 < NF) {
        if (nxt) read1(f0, SN{}, 0, std::integral_constant<int, idx / 2>{});
      }
      if constexpr (idx % 2 == 1 && idx / 2 < NL) {
        if (dma) issue1(ks0 + t + ST, sc, std::integral_constant<int, idx / 2>{});
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    static_for<NF>([&](auto qc) __attribute__((always_inline)) {
      if constexpr (decltype(qc)::value >= NM / 2) {
        if (nxt) read1(f0, SN{}, 0, qc);
      }
    });
    static_for<NL>([&](auto qc) __attribute__((always_inline)) {
      if constexpr (decltype(qc)::value >= NM / 2) {
        if (dma) issue1(ks0 + t + ST, sc, qc);
      }
    });
  };
  using YES = std::integral_constant<bool, true>;
  using NO = std::integral_constant<bool, false>;
  if (nks > 0) {
    // prologue: the DMA of steps 0 .. ST-1, then wait for step 0's
    static_for<ST>([&](auto sc) __attribute__((always_inline)) {
      if (decltype(sc)::value < nks) static_for<NL>([&](auto qc) __attribute__((always_inline)) { issue1(ks0 + decltype(sc)::value, sc, qc); });
    });
    const int later = min(ST, nks) - 1;  // steps issued after step 0
    if (ST == 3 && later == 2) wait_vm_barrier<2 * NL>();
    else if (later >= 1) wait_vm_barrier<NL>();
    else wait_vm_barrier<0>();
    static_for<NF>([&](auto qc) __attribute__((always_inline)) { read1(f0, I{}, 0, qc); });
    int t = 0;
    for (; t + 2 * ST - 1 < nks; t += ST)  // steady state: every check of the step holds
      static_for<ST>([&](auto sc) __attribute__((always_inline)) { step(t + decltype(sc)::value, sc, YES{}); });
    // fewer than 2*ST - 1 steps remain, on stages 0, 1, ..
    static_for<2 * ST - 1>([&](auto u) __attribute__((always_inline)) {
      constexpr int U = decltype(u)::value;
      if (t + U < nks) step(t + U, std::integral_constant<int, U % ST>{}, NO{});
    });
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue.  Fragment (i, j), register q: row wm*WM + 16i + 4(l/16) + q,
  // column wn*WN + 16j + (l%16) of the tile.
  const int er = 4 * (lane >> 4), ec = lane & 15;
  if (kslices > 1) {
    float* p = g.partial + (size_t)blockIdx.z * g.M * g.N;
    static_for<NM>([&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value / FN, j = decltype(ic)::value % FN;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + wm * WM + 16 * i + er + q, n = n0 + wn * WN + 16 * j + ec;
        if (m < m1 && n < g.N) p[(size_t)m * g.N + n] = acc[i][j][q];
      }
    });
    return;
  }
  if constexpr (EP == kEpGated) {
    // gate (wn = 0) and up (wn = 1) products rounded to bf16, and the rows'
    // bf16 scales, to LDS (every wave is past its last stage read: the
    // barrier orders the exchange after them); then all 256 threads take 8
    // consecutive output columns at a time and store them as 16 bytes
    constexpr int HC = BN / 2;                       // output columns of the tile
    uint16_t* sgate = (uint16_t*)st0;                // [BM][HC] bf16
    uint16_t* sup = (uint16_t*)st1;                  // [BM][HC] bf16
    float* sw = (float*)(st0 + BM * HC * 2);         // [BM] row scales
    static_assert(BM * HC * 2 + BM * 4 <= SB, "exchange buffer too small");
    __syncthreads();
    static_for<NM>([&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value / FN, j = decltype(ic)::value % FN;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        (wn ? sup : sgate)[(wm * WM + 16 * i + er + q) * HC + 16 * j + ec] = f2bf(acc[i][j][q]);
    });
    for (int r = tid; r < BM; r += 256) {
      const int m = min(m0 + r, m1 - 1);
      sw[r] = (g.row_scale != nullptr) ? rbf(g.row_scale[m]) : 1.0f;
    }
    __syncthreads();
    uint16_t* c = (uint16_t*)g.c;
    const bool vec = (((uintptr_t)c | (uintptr_t)(g.ldc * 2)) & 15u) == 0;
    for (int e = tid; e < BM * (HC / 8); e += 256) {
      const int r = e / (HC / 8), c8 = (e % (HC / 8)) * 8;
      const int m = m0 + r, n = n0 + c8;
      if (m >= m1 || n >= g.N) continue;
      const u32x4 gv = *(const u32x4*)(sgate + r * HC + c8), uv = *(const u32x4*)(sup + r * HC + c8);
      const float wr = sw[r];
      uint32_t o[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        float a0 = rbf(rbf(gelu_tanh(bf_lo(gv[h]))) * bf_lo(uv[h]));
        float a1 = rbf(rbf(gelu_tanh(bf_hi(gv[h]))) * bf_hi(uv[h]));
        if (g.row_scale != nullptr) {
          a0 = rbf(a0 * wr);
          a1 = rbf(a1 * wr);
        }
        o[h] = pack2(a0, a1);
      }
      uint16_t* dst = c + (size_t)m * g.ldc + n;
      if (vec && n + 8 <= g.N) {
        *(u32x4*)dst = u32x4{o[0], o[1], o[2], o[3]};
      } else {
        for (int h = 0; h < 8 && n + h < g.N; ++h) dst[h] = (uint16_t)(o[h / 2] >> (16 * (h & 1)));
      }
    }
    return;
  }
  static_for<NM>([&](auto ic) __attribute__((always_inline)) {
    constexpr int i = decltype(ic)::value / FN, j = decltype(ic)::value % FN;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = m0 + wm * WM + 16 * i + er + q, n = n0 + wn * WN + 16 * j + ec;
      if (m < m1 && n < g.N) {
        if constexpr (EP == kEpF32) ((float*)g.c)[(size_t)m * g.ldc + n] = acc[i][j][q];
        else ((uint16_t*)g.c)[(size_t)m * g.ldc + n] = f2bf(acc[i][j][q]);
      }
    }
  });
}

// ---- skinny GEMM (M <= 16 rows: batched decode, short prompts)
// A block owns 16*NTL output columns (B rows; with the gated epilogue the
// gate and the up rows) for all M <= 16 A rows; its NWV waves (8 for the
// 16-column products, 4 for the 64-column ones) split K into NWV ranges.
// Per k-step a wave loads one A fragment and multiplies it into NTL 16x16
// MFMA chains (A rows beyond M are clamped duplicates and are not stored).
// The wave partials meet in LDS and are summed in wave order, so there is no
// split-K reduce kernel.  Each wave requests CHK k-steps of A and B -- its
// whole K range when that fits, so one round trip -- before the first
// multiply.  NTL = 4 amortises the A fragments over 64 columns when N
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

// 1-D grid of tiles x column tiles (rounded up to a multiple of the 8 XCDs;
// ids past the live count exit), blockIdx.z = K slice.
template <int BM, int BN, int ST, int OCC, int EP>
static void launch(const GemmArgs& g, int64_t mtiles, hipStream_t st) {
  const int ncol = (EP == kEpGated) ? BN / 2 : BN;
  const int64_t nb = mtiles * ((g.N + ncol - 1) / ncol);
  dim3 grid((unsigned)(((nb + 7) / 8) * 8), 1, (unsigned)g.k_slices);
  if (g.tiles != nullptr) hipLaunchKernelGGL((gemm_kernel<BM, BN, ST, OCC, EP, true>), grid, dim3(256), 0, st, g);
  else hipLaunchKernelGGL((gemm_kernel<BM, BN, ST, OCC, EP, false>), grid, dim3(256), 0, st, g);
}

int gemm_bf16_tiles(const uint16_t* a, int64_t lda, const int32_t* a_rows, const uint16_t* b, int64_t ldb,
                    int64_t b_group_stride, int64_t pair_offset, int64_t M, int64_t N, int64_t K,
                    const int32_t* tiles, const int32_t* ntiles, int64_t max_tiles, int32_t epilogue, void* c,
                    int64_t ldc, const float* row_scale, int64_t k_slices, void* ws, int64_t ws_bytes, int tile_rows,
                    void* stream);

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
  return g4mi::gemm_bf16_tiles(a, lda, a_rows, b, ldb, b_group_stride, pair_offset, M, N, K, tiles, ntiles, max_tiles,
                               epilogue, c, ldc, row_scale, k_slices, ws, ws_bytes, 128, stream);
}

}  // extern "C"

namespace g4mi {

// g4mi_gemm_bf16 with grouped tiles of up to tile_rows (128 or 192) rows: the
// MoE prefill's expert tiles are 192 rows once most experts have more than
// 128 rows (one tile per expert, so its weights stream once, still two
// blocks per CU).
int gemm_bf16_tiles(const uint16_t* a, int64_t lda, const int32_t* a_rows, const uint16_t* b, int64_t ldb,
                    int64_t b_group_stride, int64_t pair_offset, int64_t M, int64_t N, int64_t K,
                    const int32_t* tiles, const int32_t* ntiles, int64_t max_tiles, int32_t epilogue, void* c,
                    int64_t ldc, const float* row_scale, int64_t k_slices, void* ws, int64_t ws_bytes, int tile_rows,
                    void* stream) {
  G4MI_REQUIRE(tile_rows == 128 || (tile_rows == 192 && tiles != nullptr), G4MI_EINVAL,
               "gemm: grouped tiles are 128 or 192 rows");
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
      // a wave's whole K range in one request: with 8 waves an eighth of at
      // most 12 (or 16) steps, with 4 a quarter of at most 24 (or 32)
      const dim3 grid((unsigned)((N + 15) / 16));
      const bool wide = (K / 32 + 3) / 4 > 24;
      const bool w8 = skinny_8_waves();
      const bool wide8 = (K / 32 + 7) / 8 > 12;
#define G4MI_SKINNY(E)                                                                          \
  if (w8 && wide8) hipLaunchKernelGGL((gemm_skinny_kernel<E, 1, 16, 8>), grid, dim3(512), 0, st, g); \
  else if (w8) hipLaunchKernelGGL((gemm_skinny_kernel<E, 1, 12, 8>), grid, dim3(512), 0, st, g); \
  else if (wide) hipLaunchKernelGGL((gemm_skinny_kernel<E, 1, 32>), grid, dim3(256), 0, st, g);      \
  else hipLaunchKernelGGL((gemm_skinny_kernel<E, 1, 24>), grid, dim3(256), 0, st, g);
      if (epilogue == kEpGated) { G4MI_SKINNY(kEpGated) }
      else if (epilogue == kEpF32) { G4MI_SKINNY(kEpF32) }
      else { G4MI_SKINNY(kEpBf16) }
#undef G4MI_SKINNY
    }
    return check_launch("gemm_bf16 (skinny)");
  }
  // grouped tiles are up to 128 rows (128-row kernels) or, through
  // gemm_bf16_tiles, 192; small plain M takes
  // 64-row tiles.  Two blocks per CU (2 stages) for grouped tiles and when
  // there are more tiles than CUs, else one block per CU with 3 stages.
  const bool small = tiles == nullptr && M <= 64;
  const int64_t mtiles = tiles ? max_tiles : (M + (small ? 63 : 127)) / (small ? 64 : 128);
  const int64_t ncol = epilogue == kEpGated ? 64 : 128;
  const int64_t nblocks = mtiles * ((N + ncol - 1) / ncol) * k_slices;
  G4MI_REQUIRE(mtiles * ((N + ncol - 1) / ncol) <= 2147483647 - 8, G4MI_EINVAL, "gemm: too many tiles");
  G4MI_REQUIRE(tiles == nullptr || max_tiles <= 2147483647, G4MI_EINVAL, "gemm: too many tiles");
  const int ep = (k_slices > 1) ? (int)kEpF32 : epilogue;
#define G4MI_GEMM(BM, BN, S, O)                                                 \
  if (ep == kEpGated) launch<BM, BN, S, O, kEpGated>(g, mtiles, st);            \
  else if (ep == kEpF32) launch<BM, BN, S, O, kEpF32>(g, mtiles, st);           \
  else launch<BM, BN, S, O, kEpBf16>(g, mtiles, st);
  if (small) {
    G4MI_GEMM(64, 128, 3, 1)
  } else if (tiles != nullptr && tile_rows == 192) {
    G4MI_GEMM(192, 128, 2, 2)
  } else if (tiles != nullptr || nblocks > 256) {
    G4MI_GEMM(128, 128, 2, 2)
  } else {
    G4MI_GEMM(128, 128, 3, 1)
  }
#undef G4MI_GEMM
  if (k_slices > 1) {
    const int64_t mn = M * N;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st, (const float*)ws,
                       (int)k_slices, mn, (int)N, c, ldc, epilogue == kEpF32 ? 1 : 0);
  }
  return check_launch("gemm_bf16");
}

}  // namespace g4mi

extern "C" {

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
  if (skinny_8_waves()) {
    if ((K / 32 + 7) / 8 > 12) hipLaunchKernelGGL((gemm_skinny_kernel<kEpBf16, 1, 16, 8>), grid, dim3(512), 0, st, g);
    else hipLaunchKernelGGL((gemm_skinny_kernel<kEpBf16, 1, 12, 8>), grid, dim3(512), 0, st, g);
  } else if ((K / 32 + 3) / 4 > 24) {
    hipLaunchKernelGGL((gemm_skinny_kernel<kEpBf16, 1, 32>), grid, dim3(256), 0, st, g);
  } else {
    hipLaunchKernelGGL((gemm_skinny_kernel<kEpBf16, 1, 24>), grid, dim3(256), 0, st, g);
  }
  return check_launch("gemm_bf16_segments");
}

// Host-only diagnostics: the tile that block bid of a grid sized for
// max_tiles row tiles runs when mtiles of them are live, as (tx, ty) in
// out[2 bid], out[2 bid + 1], or (-1, -1) for a block that exits.
int g4mi_selftest_tile_order(int32_t mtiles, int32_t max_tiles, int32_t ncol_tiles, int32_t grouped,
                             int32_t* out, int64_t out_len) {
  G4MI_REQUIRE(out != nullptr, G4MI_EINVAL, "selftest_tile_order: null output");
  G4MI_REQUIRE(mtiles >= 0 && max_tiles >= 1 && mtiles <= max_tiles && ncol_tiles >= 1, G4MI_EINVAL,
               "selftest_tile_order: need 0 <= mtiles <= max_tiles and ncol_tiles >= 1");
  const int64_t nb = (int64_t)max_tiles * ncol_tiles, grid = (nb + 7) / 8 * 8;
  G4MI_REQUIRE(grid <= 2147483647 && out_len >= 2 * grid, G4MI_EINVAL, "selftest_tile_order: output too small");
  for (int64_t b = 0; b < grid; ++b) {
    int tx = -1, ty = -1;
    if (!tile_of((int)b, mtiles, ncol_tiles, tx, ty, grouped != 0)) tx = ty = -1;
    out[2 * b] = tx;
    out[2 * b + 1] = ty;
  }
  return 0;
}

}  // extern "C"
