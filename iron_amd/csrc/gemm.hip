// bf16 GEMM on MFMA for prefill: C[M][N] = epilogue(sum_k A[m][k] * B[n][k]).
//
// "NT" form: A (M, K) and B (N, K) are both K-contiguous, which is how
// nn.Linear weights are stored (out_features, in_features) and what the MFMA
// operands want: with v_mfma_f32_32x32x16_bf16 every lane feeds 8 consecutive
// k of one row (lane l -> row l%32, k (l/32)*8..+8), so each operand fragment
// is a single 16-byte LDS read. Other layouts are reduced to this one on the
// host (B row-major (K, N) through a transpose, C column-major by swapping the
// operands: C^T = B A^T).
//
// Tiles: a workgroup of WMW x WNW waves owns a (WMW*TI*32) x (WNW*TJ*32)
// output tile; each wave owns TI x TJ MFMA tiles of 32x32. gemm_launch picks
// one of five shapes with a cost model: 256x256 (8 waves of 64x128), 256x192
// (8 waves of 64x96, when it divides N), 256x128 (8 waves of 64x64, 3 stages),
// 128x128 with 8 waves of 64x32 (one workgroup per CU, 3 steps of look-ahead)
// and 128x128 with 4 waves of 64x64 (two workgroups per CU). Shapes too small
// to give every CU a 128x128 tile take 64x64 or 128x64 tiles (4 waves).
// Bigger tiles fetch fewer bytes per flop: at ~64 B/clk of L2->CU fill per CU,
// a 128x128x64 step needs as many cycles to fill as its MFMAs take, a 256x256
// step half as many. Two waves per SIMD hide each
// other's LDS and barrier waits, which matters most when each CU has a single
// workgroup.
//
// K advances 64 per step through an NS-stage LDS ring filled by LDS-direct
// loads (buffer_load_dwordx4 ... lds, load_lds16): they write LDS directly, with no VGPR staging
// and no ds_write (ds_write_b128 sustains ~73 B/clk per CU against ~205 B/clk
// for ds_read_b128, and was the main loop's bottleneck). A stage holds the A
// rows then the B rows, 128 B (64 bf16) each, in 1 KiB blocks of 8 rows; the
// lane that lands on (row, slot) fetches chunk slot ^ ((row / 2) % 8), so
// the 16-byte chunk c of row r sits at slot c ^ ((r / 2) % 8) (see swz).
// Rows past M or N load row M-1 or N-1 instead: they only feed outputs that
// are never stored.
//
// One barrier per step, placed before the step's last k-slice's MFMAs: those
// MFMAs run while the next step's first fragments are read (the gemm_nt
// kernel). Fragments are double-buffered in registers across the four 16-deep
// k-slices of a step.
// Tile order is XCD-aware (tile_coords): workgroup b runs on XCD b % 8, and
// the tiles an XCD runs share A row blocks and B column blocks in its L2.
// Epilogue: round to bf16, then activation and clamp (the flm.GEMM order),
// staged through LDS so global stores are 16-byte and row-contiguous.
#include <algorithm>

#include "iron_common.hpp"
#include "trace.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));

constexpr int BK = 64;
// Buffer offsets are 32-bit: a tile's rows (at most 256) times K times 2 bytes must stay below 2^31.
constexpr int kMaxK = 1 << 21;


constexpr int kChunks = BK / 8;  // 16-byte chunks per LDS row
constexpr int kSplitTile = 128;  // tile edge the split-K policy counts in
// Epilogue of the fused SwiGLU GEMM (iron_gemm_bf16_nt_swiglu); not part of the
// public enum: B rows come in 64-row blocks alternating gate / up.
constexpr int kEpiSwigluPair = 100;

// bf16 of x for the output stage: round to nearest even, or toward zero
// (mantissa truncation, flm.GEMM's "floor" conversion); NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t out_bf16(float x, int toward_zero) {
  if (!toward_zero) return f32_to_bf16(x);
  const uint32_t u = __float_as_uint(x);
  return static_cast<uint16_t>(x != x ? (u >> 16) | 0x40u : u >> 16);
}

struct GemmArgs {
  const uint16_t* A;  // (M, K)
  const uint16_t* B;  // (N, K)
  uint16_t* C;        // (M, N), row stride ldc
  int M, N, K;
  long long ldc;
  int epi;
  int clamp;
  float lo, hi;
  float* partial;  // split-K: fp32 (splits, M, N) partial sums instead of C
  int splits;      // K ranges (1 = no split)
  // int4-g32 B (gemm_i4_kernel): codes (N, K/2), low nibble = even k; bf16
  // scales (N, K/32); is_signed: two's-complement codes (else unsigned)
  const uint8_t* codes;
  const uint16_t* scales;
  int is_signed;
  int toward_zero;  // output-stage conversions truncate instead of rounding to nearest even
  void* trace;      // phase trace records (trace.hpp), read by the traced instance only
};

// Splits an entry point's epilogue code into the activation (a.epi) and the
// IRON_EPI_ROUND_TOWARD_ZERO flag (a.toward_zero).
static void set_epilogue(GemmArgs& a, int epilogue) {
  a.toward_zero = (epilogue & IRON_EPI_ROUND_TOWARD_ZERO) != 0;
  a.epi = epilogue & ~IRON_EPI_ROUND_TOWARD_ZERO;
}

// G_: tile order by XCD regions (tile_coords).
template <int WMW_, int WNW_, int TI_, int TJ_, int NS_, bool G_ = false>
struct Tile {
  static constexpr int WMW = WMW_, WNW = WNW_, TI = TI_, TJ = TJ_, NS = NS_;
  static constexpr bool G = G_;
  static constexpr int kWaves = WMW * WNW, kThreads = 64 * kWaves;
  static constexpr int BM = WMW * TI * 32, BN = WNW * TJ * 32;
  static constexpr int kPerWave = (BM + BN) / 8 / kWaves;  // 1 KiB blocks each wave loads per step
  static constexpr int kStage = (BM + BN) * kChunks;       // 16-byte slots per stage
  static_assert((BM + BN) / 8 % kWaves == 0, "a stage's blocks must split evenly over the waves");
  static_assert(BM * BN * 2 <= NS * kStage * 16, "the bf16 C tile must fit in the stages' LDS");
};
using TileL = Tile<4, 2, 2, 4, 2, true>;   // 256x256, 8 waves of 64x128, 128 KiB
using TileM = Tile<4, 2, 2, 2, 3, true>;   // 256x128, 8 waves of 64x64, 3 stages (144 KiB; one workgroup per CU either way)
using TileS = Tile<2, 4, 2, 1, 4>;         // 128x128, 8 waves of 64x32, 128 KiB, 3 steps ahead
using TileS2 = Tile<2, 2, 2, 2, 2>;        // 128x128, 4 waves of 64x64, 64 KiB: two workgroups per CU
using TileL3 = Tile<4, 2, 2, 3, 2, true>;  // 256x192, 8 waves of 64x96, 112 KiB: N = 3072 in 16 tiles
using Tile64 = Tile<2, 2, 1, 1, 4>;        // 64x64, 4 waves of 32x32, 64 KiB: shapes too small for 128x128
using Tile128x64 = Tile<2, 2, 2, 1, 4>;    // 128x64, 4 waves of 64x32, 96 KiB

// A 16-byte LDS access of 16 lanes covers all 64 banks once when their 16
// consecutive rows use 16 distinct (row parity, slot) pairs: the slot is
// chunk ^ ((row / 2) % 8). (chunk ^ (row % 8) repeats every 8 rows, which put
// rows r and r + 8 on the same banks: a 2-way conflict on every fragment read.)
__device__ __forceinline__ int swz(int row, int chunk) { return row * kChunks + (chunk ^ ((row >> 1) & 7)); }

// Wait until at most N of this wave's global loads are outstanding, then
// barrier. (__syncthreads would wait for all of them.) The memory clobber
// keeps LDS reads of the next stage below the barrier.
template <int N>
__device__ __forceinline__ void wait_loads_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Epilogue shared by the GEMM kernels. Split-K: raw fp32 sums straight from
// the accumulators. Otherwise the C tile goes through LDS as bf16 [BM][BN]
// (every wave must be done reading its last stage) for 16-byte row stores.
template <class T>
__device__ __forceinline__ void store_tile(const GemmArgs& a, const f32x16_t (&acc)[T::TI][T::TJ], u32x4v* smem,
                                           int m0, int n0, int kb, int wm, int wn, int lane, int tid) {
  constexpr int BM = T::BM, BN = T::BN, TI = T::TI, TJ = T::TJ;
  if (a.partial) {  // split-K: raw fp32 sums straight from the accumulators
    float* P = a.partial + static_cast<size_t>(kb) * a.M * a.N;
    if (m0 + BM <= a.M && n0 + BN <= a.N) {  // the whole tile is inside (uniform): no per-element tests
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int gm = m0 + wm * TI * 32 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            const int gn = n0 + wn * TJ * 32 + j * 32 + (lane & 31);
            P[static_cast<size_t>(gm) * a.N + gn] = acc[i][j][v];
          }
      return;
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int gm = m0 + wm * TI * 32 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          const int gn = n0 + wn * TJ * 32 + j * 32 + (lane & 31);
          if (gm < a.M && gn < a.N) P[static_cast<size_t>(gm) * a.N + gn] = acc[i][j][v];
        }
    return;
  }

  // epilogue through LDS: C tile as bf16 [BM][BN]
  __syncthreads();  // every wave is done reading the last stage
  uint16_t* Cs = reinterpret_cast<uint16_t*>(smem);
  const bool swiglu = a.epi == kEpiSwigluPair;
  // The epilogue's options are uniform: branch once on them, not per element
  // (per-element tests of the activation, clamp and rounding mode cost more
  // than the conversions, and this loop runs with the CU otherwise idle).
  if ((swiglu || (a.epi == EPI_NONE && !a.clamp)) && !a.toward_zero) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = wm * TI * 32 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          const int col = wn * TJ * 32 + j * 32 + (lane & 31);
          Cs[row * BN + col] = f32_to_bf16(acc[i][j][v]);
        }
  } else {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = wm * TI * 32 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          const int col = wn * TJ * 32 + j * 32 + (lane & 31);
          float x = acc[i][j][v];
          if (!swiglu && (a.epi != EPI_NONE || a.clamp)) {
            x = bf16_to_f32(out_bf16(x, a.toward_zero));
            x = apply_epilogue(x, a.epi);
            if (a.clamp) x = fminf(fmaxf(x, a.lo), a.hi);
          }
          Cs[row * BN + col] = out_bf16(x, a.toward_zero);
        }
  }
  __syncthreads();
  if (swiglu) {
    // Column blocks 2p and 2p+1 of 64 hold gate and up of features
    // n0/2 + 64p .. + 63: h = bf16(silu(g) * u) of the bf16-rounded g and u,
    // as iron_silu_mul on separate gate and up GEMM outputs. C is (M, N/2).
    constexpr int CH = BN / 16;  // 8-feature chunks per output row
    const int F = a.N / 2;
    const bool full_f = (n0 / 2 + BN / 2 <= F) && (a.ldc % 8 == 0);
    auto h_chunk = [&](int row, int c) {  // 8 features of one row: silu(g) * u, packed bf16
      const int gcol = (c / 8) * 128 + (c % 8) * 8;
      const uint4 gv = reinterpret_cast<const uint4*>(Cs)[(row * BN + gcol) / 8];
      const uint4 uv = reinterpret_cast<const uint4*>(Cs)[(row * BN + gcol + 64) / 8];
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        h[e] = cvt_pk_bf16(silu_f32(lo_bf16(gw[e])) * lo_bf16(uw[e]), silu_f32(hi_bf16(gw[e])) * hi_bf16(uw[e]));
      return make_uint4(h[0], h[1], h[2], h[3]);
    };
    if (full_f && m0 + BM <= a.M) {  // the whole tile is inside H (uniform)
#pragma unroll
      for (int i = 0; i < (BM * CH) / T::kThreads; ++i) {
        const int id = tid + i * T::kThreads, row = id / CH, c = id % CH;
        *reinterpret_cast<uint4*>(a.C + static_cast<size_t>(m0 + row) * a.ldc + n0 / 2 + c * 8) = h_chunk(row, c);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < (BM * CH) / T::kThreads; ++i) {
      const int id = tid + i * T::kThreads, row = id / CH, c = id % CH;
      const int gcol = (c / 8) * 128 + (c % 8) * 8;
      const int gm = m0 + row, gf = n0 / 2 + c * 8;
      if (gm >= a.M || gf >= F) continue;
      const uint4 gv = reinterpret_cast<const uint4*>(Cs)[(row * BN + gcol) / 8];
      const uint4 uv = reinterpret_cast<const uint4*>(Cs)[(row * BN + gcol + 64) / 8];
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        h[e] = cvt_pk_bf16(silu_f32(lo_bf16(gw[e])) * lo_bf16(uw[e]), silu_f32(hi_bf16(gw[e])) * hi_bf16(uw[e]));
      uint16_t* dst = a.C + static_cast<size_t>(gm) * a.ldc + gf;
      if (full_f) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(h[0], h[1], h[2], h[3]);
      } else {
        for (int q = 0; q < 8; ++q)
          if (gf + q < F) dst[q] = static_cast<uint16_t>(h[q / 2] >> (16 * (q & 1)));
      }
    }
    return;
  }
  const bool full_n = (n0 + BN <= a.N) && (a.ldc % 8 == 0);
  if (full_n && m0 + BM <= a.M) {  // the whole tile is inside C (uniform)
#pragma unroll
    for (int i = 0; i < (BM * BN / 8) / T::kThreads; ++i) {
      const int id = tid + i * T::kThreads, row = id / (BN / 8), c = id % (BN / 8);
      *reinterpret_cast<uint4*>(a.C + static_cast<size_t>(m0 + row) * a.ldc + n0 + c * 8) =
          reinterpret_cast<const uint4*>(Cs)[row * (BN / 8) + c];
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < (BM * BN / 8) / T::kThreads; ++i) {
    const int id = tid + i * T::kThreads, row = id / (BN / 8), c = id % (BN / 8);
    const int gm = m0 + row, gn = n0 + c * 8;
    if (gm >= a.M || gn >= a.N) continue;
    const uint4 v = reinterpret_cast<const uint4*>(Cs)[row * (BN / 8) + c];
    uint16_t* dst = a.C + static_cast<size_t>(gm) * a.ldc + gn;
    if (full_n) {
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
      for (int q = 0; q < 8; ++q)
        if (gn + q < a.N) dst[q] = e[q];
    }
  }
}

// Workgroup b runs on XCD b % 8. Default order: XCD x takes the x-th eighth of the (tiles x K ranges)
// sequence, M fastest, so consecutive tiles along M (which share one B column block) share an L2.
// Region order (T::G, no K split, a tile grid that divides into 8 regions): XCD x owns a px x py
// region of the tile grid, px * py = 8, chosen to minimise the A rows plus B rows the region reads,
// and runs it in groups of 4 tile rows, so the tiles resident together on an XCD (32, one per CU)
// share 4 A row blocks and a few B column blocks in its L2. For the 3968-token down projection
// (256x128 tiles, 16 x 16) this cuts what the L2s fetch per launch from 791 to ~330 MB.
template <class T>
__device__ __forceinline__ void tile_coords(const GemmArgs& a, int b, int& kb, int& tm, int& tn) {
  const int tiles_m = (a.M + T::BM - 1) / T::BM, tiles_n = (a.N + T::BN - 1) / T::BN;
  const int nt = tiles_m * tiles_n * a.splits;
  if (T::G && a.splits == 1) {
    int px = 0, best = 1 << 30;
    for (int q = 1; q <= 8; q *= 2)
      if (tiles_m % q == 0 && tiles_n % (8 / q) == 0) {
        const int c = tiles_m / q * T::BM + tiles_n / (8 / q) * T::BN;
        if (c < best) best = c, px = q;
      }
    if (px) {
      constexpr int GM = 4;
      const int RM = tiles_m / px, RN = tiles_n / (8 / px), x = b % 8, i = b / 8;
      const int g = i / (GM * RN), j = i % (GM * RN), gm = min(GM, RM - g * GM);
      kb = 0;
      tm = (x % px) * RM + g * GM + j % gm;
      tn = (x / px) * RN + j / gm;
      return;
    }
  }
  int t = b;
  if (nt % 8 == 0) t = (t % 8) * (nt / 8) + t / 8;
  kb = t / (tiles_m * tiles_n);
  t %= tiles_m * tiles_n;
  tm = t % tiles_m, tn = t / tiles_m;
}

// TR: the instance launched while a phase trace is armed (trace.hpp); the
// others carry no trace code. Trace points: 0 start, 1 first stage in LDS,
// 2-4 after a quarter, half and three quarters of the K steps, 5 tile stored.
template <class T, bool TR>
__global__ __launch_bounds__(T::kThreads) void gemm_nt_kernel(GemmArgs a) {
  constexpr int BM = T::BM, BN = T::BN, TI = T::TI, TJ = T::TJ, NS = T::NS, PW = T::kPerWave;
  __shared__ u32x4v smem[NS * T::kStage];
  void* const trace = TR ? a.trace : nullptr;
  unsigned long long t_start = 0;
  if constexpr (TR) t_start = trace_clock();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / T::WNW, wn = wave % T::WNW;

  int kb, tm, tn;
  tile_coords<T>(a, blockIdx.x, kb, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = a.K / BK / a.splits;  // steps in this workgroup's K range

  // The PW blocks this wave loads each step: block b < BM/8 is rows 8b..8b+7
  // of A, the rest are rows of B, through buffer resources based at the tile's
  // first A row and first B row (load_lds16). off[j]: byte offset of this lane's
  // chunk at the range's first step.
  const i32x4v rsrc_a = buffer_rsrc(a.A + static_cast<size_t>(m0) * a.K);
  const i32x4v rsrc_b = buffer_rsrc(a.B + static_cast<size_t>(n0) * a.K);
  unsigned off[PW];
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int b = wave * PW + j;
    const bool is_a = b < BM / 8;
    const int row = (is_a ? b : b - BM / 8) * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ ((row >> 1) & 7);
    const int r = is_a ? min(m0 + row, a.M - 1) - m0 : min(n0 + row, a.N - 1) - n0;
    off[j] = static_cast<unsigned>((r * a.K + kb * nk * BK + chunk * 8) * 2);
  }
  auto issue = [&](int step) {
#pragma unroll
    for (int j = 0; j < PW; ++j)
      load_lds16(wave * PW + j < BM / 8 ? rsrc_a : rsrc_b, off[j] + step * BK * 2,
                 smem + (step % NS) * T::kStage + (wave * PW + j) * 64);
  };

  f32x16_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  bf16x8_t fa[2][TI], fb[2][TJ];
  auto read_frags = [&](int set, int stage, int kk) {
    const u32x4v* As = smem + stage * T::kStage;
    const u32x4v* Bs = As + BM * kChunks;
    const int c = kk * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TI; ++i)
      fa[set][i] = __builtin_bit_cast(bf16x8_t, As[swz(wm * TI * 32 + i * 32 + (lane & 31), c)]);
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      fb[set][j] = __builtin_bit_cast(bf16x8_t, Bs[swz(wn * TJ * 32 + j * 32 + (lane & 31), c)]);
  };

  // prologue: steps 0..NS-2 in flight, wait for step 0, first fragments
#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < nk) issue(p);
  trace_write(trace, kTraceGemm, blockIdx.x, 0, t_start);
  if (NS - 1 < nk)
    wait_loads_barrier<PW * (NS - 2)>();
  else
    wait_loads_barrier<0>();
  read_frags(0, 0, 0);
  trace_stamp(trace, kTraceGemm, blockIdx.x, 1);

  // One step; LAST: the range's last step (no barrier, no next fragments). The
  // last step is peeled off so that the other steps' final k-slice has one
  // path into its MFMAs, and the compiler's LDS waits there count exactly.
  auto step = [&](int s, auto last_tag) {
    constexpr bool LAST = decltype(last_tag)::value;
    // the stage read in step s-1: every wave passed the barrier after its last read of it
    if (s + NS - 1 < nk) issue(s + NS - 1);
    // How the compiler interleaves the next slice's fragment reads with this
    // slice's MFMAs sets how much LDS latency is exposed; its DS/MFMA
    // interleave strategy 0 measured 2-4% faster on every shape than its default.
    __builtin_amdgcn_iglp_opt(0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int cur = kk & 1, nxt = cur ^ 1;
      if (kk + 1 < BK / 16) {
        read_frags(nxt, s % NS, kk + 1);
      } else if constexpr (!LAST) {
        // The step's barrier comes before its last k-slice's MFMAs, so the next
        // step's first fragment reads are in flight while those MFMAs run. This
        // wave's reads of stage s % NS (which the next step's loads refill) have
        // all returned: the last slice's fragments are waited for first, after
        // the previous slice's MFMAs (the scheduling fence keeps them above it).
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // steps s+2..min(s+NS-1, nk-1) may stay in flight
        if (s + NS - 1 < nk)
          wait_loads_barrier<PW * (NS - 2)>();
        else
          wait_loads_barrier<0>();
        read_frags(nxt, (s + 1) % NS, 0);
      }
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
    }
  };
  for (int s = 0; s + 1 < nk; ++s) {
    step(s, std::false_type{});
    if constexpr (TR) {
      if (4 * (s + 1) == nk || 2 * (s + 1) == nk || 4 * (s + 1) == 3 * nk)
        trace_stamp(trace, kTraceGemm, blockIdx.x, 4 * (s + 1) == nk ? 2 : 2 * (s + 1) == nk ? 3 : 4);
    }
  }
  step(nk - 1, std::true_type{});

  store_tile<T>(a, acc, smem, m0, n0, kb, wm, wn, lane, tid);
  trace_stamp(trace, kTraceGemm, blockIdx.x, 5);
}

// ---------------------------------------------------------------------------
// int4-g32 weights dequantized in the GEMM's prologue: C = epi(A . deq(B)^T),
// deq(B)[n][k] = bf16(q[n][k] * s[n][k / 32]) (the product is exact in fp32,
// rounded once to nearest-even), q two's-complement or unsigned nibbles, low
// nibble first along K. Per step the workgroup fetches, by LDS-direct loads,
// the A tile (as the bf16 kernel) plus the B codes (BN x 32 B) and scales
// (BN x 4 B), then dequantizes the NEXT step's B tile once for all its waves
// into one of two bf16 tiles (same swizzled layout as a bf16 B stage) after
// issuing the current step's MFMAs, which read the other tile. The MFMA chain is the bf16 kernel's, so the
// result is bit-identical to iron_gemm_bf16_nt on the dequantized weights.
// Dequantization: (n ^ 8) (signed) or n via a byte mask, v_cvt_f32_ubyte,
// one FMA with the scale (q*s = (q+8)*s - 8s exactly), v_cvt_pk_bf16_f32.
template <int WMW_, int WNW_, int TI_, int TJ_, int NS_>
struct TileI4 {
  static constexpr int WMW = WMW_, WNW = WNW_, TI = TI_, TJ = TJ_, NS = NS_;
  static constexpr int kWaves = WMW * WNW, kThreads = 64 * kWaves;
  static constexpr int BM = WMW * TI * 32, BN = WNW * TJ * 32;
  static constexpr int kABlocks = BM / 8;    // 1 KiB blocks of 8 A rows
  static constexpr int kCBlocks = BN / 32;   // 1 KiB blocks of 32 code rows (32 B each)
  static constexpr int kSBlocks = BN / 64;   // 256 B blocks of 64 scale pairs
  static constexpr int kSlots = kABlocks + kCBlocks + kSBlocks;
  static constexpr int kPerWave = (kSlots + kWaves - 1) / kWaves;  // loads per wave per step (padded)
  // LDS (bytes): NS stages of [A | codes | scales], then 2 bf16 B tiles, then a dummy KiB
  static constexpr int kStageBytes = BM * 128 + BN * 32 + BN * 4;
  static constexpr int kBbfOff = NS * kStageBytes;
  static constexpr int kDummyOff = kBbfOff + 2 * BN * 128;
  static constexpr int kLds = kDummyOff + 1024;
  static_assert(NS >= 3, "the next step's codes must be resident one step ahead");
  static_assert(BN * 4 == kThreads, "one 16-weight quarter row per thread");
  static_assert(kLds <= 160 * 1024 && BM * BN * 2 <= kLds, "LDS budget");
};
using TileI4S = TileI4<2, 4, 2, 1, 4>;  // 128x128, 8 waves of 64x32
using TileI4M = TileI4<4, 2, 2, 2, 3>;  // 256x128, 8 waves of 64x64

// 8 int4 codes of one 32-bit word -> 8 bf16 weights (4 words, k order).
__device__ __forceinline__ u32x4v dequant8(uint32_t w, float s, bool is_signed) {
  const uint32_t x = is_signed ? (w ^ 0x88888888u) : w;  // signed: n ^ 8 = q + 8
  uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
  // hide the known-zero bits, so each byte converts with one v_cvt_f32_ubyteN
  asm volatile("" : "+v"(lo), "+v"(hi));
  const float off = is_signed ? -8.f * s : 0.f;
  float v[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    v[2 * b] = fmaf(static_cast<float>((lo >> (8 * b)) & 0xFFu), s, off);      // element 2b (low nibble)
    v[2 * b + 1] = fmaf(static_cast<float>((hi >> (8 * b)) & 0xFFu), s, off);  // element 2b + 1
  }
  return u32x4v{cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3]), cvt_pk_bf16(v[4], v[5]), cvt_pk_bf16(v[6], v[7])};
}

template <class T>
__global__ __launch_bounds__(T::kThreads) void gemm_i4_kernel(GemmArgs a) {
  constexpr int BM = T::BM, BN = T::BN, TI = T::TI, TJ = T::TJ, NS = T::NS, PW = T::kPerWave;
  __shared__ u32x4v smem[T::kLds / 16];
  unsigned char* lds = reinterpret_cast<unsigned char*>(smem);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / T::WNW, wn = wave % T::WNW;

  const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
  const int nt = tiles_m * tiles_n * a.splits;
  int t = blockIdx.x;
  if (nt % 8 == 0) t = (t % 8) * (nt / 8) + t / 8;
  const int kb = t / (tiles_m * tiles_n);
  t %= tiles_m * tiles_n;
  const int tm = t % tiles_m, tn = t / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = a.K / BK / a.splits;
  const int step0 = kb * nk;  // first K step of this workgroup's range

  // Load slots: A blocks, then code blocks, then scale blocks, then dummies
  // (every wave issues exactly PW loads per step, so one vmcnt count fits all).
  const unsigned char* src[PW];
  int dst[PW], kind[PW];  // kind: 0 A (16 B/lane, +128 B per step), 1 codes (16 B, +32 B), 2 scales (4 B, +4 B), 3 dummy
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int slot = wave * PW + j;
    if (slot < T::kABlocks) {
      const int row = slot * 8 + (lane >> 3), chunk = (lane & 7) ^ ((row >> 1) & 7);
      src[j] = reinterpret_cast<const unsigned char*>(a.A + static_cast<size_t>(min(m0 + row, a.M - 1)) * a.K +
                                                      static_cast<size_t>(step0) * BK + chunk * 8);
      dst[j] = slot * 1024;
      kind[j] = 0;
    } else if (slot < T::kABlocks + T::kCBlocks) {
      const int c = slot - T::kABlocks, row = c * 32 + (lane >> 1);
      src[j] = a.codes + static_cast<size_t>(min(n0 + row, a.N - 1)) * (a.K / 2) + static_cast<size_t>(step0) * 32 +
               (lane & 1) * 16;
      dst[j] = BM * 128 + c * 1024;
      kind[j] = 1;
    } else if (slot < T::kSlots) {
      const int c = slot - T::kABlocks - T::kCBlocks, row = c * 64 + lane;
      src[j] = reinterpret_cast<const unsigned char*>(a.scales + static_cast<size_t>(min(n0 + row, a.N - 1)) *
                                                                    (a.K / 32) + static_cast<size_t>(step0) * 2);
      dst[j] = BM * 128 + BN * 32 + c * 256;
      kind[j] = 2;
    } else {
      src[j] = reinterpret_cast<const unsigned char*>(a.A) + (lane & 7) * 16;  // first 128 B of A (K >= 64)
      dst[j] = 0;
      kind[j] = 3;
    }
  }
  auto issue = [&](int step) {
    unsigned char* st = lds + (step % NS) * T::kStageBytes;
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      if (kind[j] == 2)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const unsigned*>(src[j] + step * 4),
                                         reinterpret_cast<unsigned*>(st + dst[j]), 4, 0, 0);
      else if (kind[j] == 3)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const unsigned*>(src[j]),
                                         reinterpret_cast<unsigned*>(lds + T::kDummyOff), 16, 0, 0);
      else
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const unsigned*>(src[j] + step * (kind[j] == 0 ? 128 : 32)),
                                         reinterpret_cast<unsigned*>(st + dst[j]), 16, 0, 0);
    }
  };
  // Thread -> quarter row of the B tile: row tid / 4, k 16 (tid % 4) .. + 16.
  const int dq_row = tid >> 2, dq_q = tid & 3;
  // The code and scale reads are inline assembly with their own lgkmcnt wait:
  // as plain loads, the compiler made them wait vmcnt(0) for every LDS-direct
  // load in flight (it cannot tell the stages apart).
  auto dequant = [&](int step) {
    const unsigned st = static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds)) + (step % NS) * T::kStageBytes;
    const unsigned ca = st + BM * 128 + dq_row * 32 + dq_q * 8;
    const unsigned sa = st + BM * 128 + BN * 32 + dq_row * 4 + (dq_q >> 1) * 2;
    u32x2v w;
    unsigned s16;
    asm volatile("ds_read_b64 %0, %2\n\tds_read_u16 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(w), "=&v"(s16)
                 : "v"(ca), "v"(sa));
    const float sc = __builtin_bit_cast(float, s16 << 16);
    u32x4v* bt = reinterpret_cast<u32x4v*>(lds + T::kBbfOff + (step & 1) * BN * 128);
    bt[swz(dq_row, 2 * dq_q)] = dequant8(w.x, sc, a.is_signed);
    bt[swz(dq_row, 2 * dq_q + 1)] = dequant8(w.y, sc, a.is_signed);
  };

  f32x16_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // prologue: steps 0..NS-2 in flight; step 0 resident; its B tile dequantized
#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < nk) issue(p);
  if (NS - 1 < nk)
    wait_loads_barrier<PW * (NS - 2)>();
  else
    wait_loads_barrier<0>();
  dequant(0);

  for (int s = 0; s < nk; ++s) {
    // step s+1 resident (steps s+2..min(s+NS-2, nk-1) may stay in flight); the
    // barrier also publishes the B tile of step s and retires every read of
    // the stage and B tile used by step s-1
    if (s + NS - 2 < nk)
      wait_loads_barrier<PW * (NS - 3)>();
    else
      wait_loads_barrier<0>();
    if (s + NS - 1 < nk) issue(s + NS - 1);
    const u32x4v* As = reinterpret_cast<const u32x4v*>(lds + (s % NS) * T::kStageBytes);
    const u32x4v* Bs = reinterpret_cast<const u32x4v*>(lds + T::kBbfOff + (s & 1) * BN * 128);
    bf16x8_t fa[2][TI], fb[2][TJ];
    auto frags = [&](int set, int kk) {
      const int c = kk * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < TI; ++i)
        fa[set][i] = __builtin_bit_cast(bf16x8_t, As[swz(wm * TI * 32 + i * 32 + (lane & 31), c)]);
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        fb[set][j] = __builtin_bit_cast(bf16x8_t, Bs[swz(wn * TJ * 32 + j * 32 + (lane & 31), c)]);
    };
    frags(0, 0);
    __builtin_amdgcn_iglp_opt(0);  // as in gemm_nt_kernel: 2.6-3.5% faster
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int cur = kk & 1, nxt = cur ^ 1;
      if (kk + 1 < BK / 16) frags(nxt, kk + 1);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
    }
    // the next step's B tile, dequantized while this step's MFMAs execute
    if (s + 1 < nk) dequant(s + 1);
  }
  store_tile<T>(a, acc, smem, m0, n0, kb, wm, wn, lane, tid);
}

// Split-K merge: C = clamp(act(bf16(sum_kb partial[kb]))), the same epilogue
// order as the single-pass kernel. One thread per output element.
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(GemmArgs a) {
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  const long long mn = static_cast<long long>(a.M) * a.N;
  if (t >= mn) return;
  float x = 0.f;
  for (int kb = 0; kb < a.splits; ++kb) x += a.partial[kb * mn + t];
  if (a.epi != EPI_NONE || a.clamp) {
    x = bf16_to_f32(out_bf16(x, a.toward_zero));
    x = apply_epilogue(x, a.epi);
    if (a.clamp) x = fminf(fmaxf(x, a.lo), a.hi);
  }
  const long long m = t / a.N, n = t % a.N;
  a.C[m * a.ldc + n] = out_bf16(x, a.toward_zero);
}

// The same merge, 8 outputs per thread: 16-byte loads of every K range issued
// up front (at most 8 ranges; clamped indexes, the extra ones dropped by
// selects) and one 16-byte store. The sums run over the ranges in the same
// order as above, so the results are identical. Needs N % 8 == 0, ldc % 8 == 0,
// a 16-byte aligned C and M * N / 8 < 2^31 (checked on the host).
__global__ __launch_bounds__(256) void gemm_splitk_reduce8_kernel(GemmArgs a) {
  const int gpr = a.N >> 3;  // 8-output groups per row
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= a.M * gpr) return;
  const int m = t / gpr, c = t - m * gpr;
  const size_t mn4 = static_cast<size_t>(a.M) * a.N / 4;
  const float4* p = reinterpret_cast<const float4*>(a.partial) + (static_cast<size_t>(m) * a.N >> 2) + 2 * c;
  float4 u[8], v[8];
#pragma unroll
  for (int kb = 0; kb < 8; ++kb) {
    const float4* q = p + static_cast<size_t>(min(kb, a.splits - 1)) * mn4;
    u[kb] = q[0];
    v[kb] = q[1];
  }
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < 8; ++kb) {
    const bool live = kb < a.splits;
    x[0] = live ? x[0] + u[kb].x : x[0];
    x[1] = live ? x[1] + u[kb].y : x[1];
    x[2] = live ? x[2] + u[kb].z : x[2];
    x[3] = live ? x[3] + u[kb].w : x[3];
    x[4] = live ? x[4] + v[kb].x : x[4];
    x[5] = live ? x[5] + v[kb].y : x[5];
    x[6] = live ? x[6] + v[kb].z : x[6];
    x[7] = live ? x[7] + v[kb].w : x[7];
  }
  uint32_t h[4];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (a.epi != EPI_NONE || a.clamp) {
      x[e] = bf16_to_f32(out_bf16(x[e], a.toward_zero));
      x[e] = apply_epilogue(x[e], a.epi);
      if (a.clamp) x[e] = fminf(fmaxf(x[e], a.lo), a.hi);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    h[e] = static_cast<uint32_t>(out_bf16(x[2 * e], a.toward_zero)) |
           (static_cast<uint32_t>(out_bf16(x[2 * e + 1], a.toward_zero)) << 16);
  *reinterpret_cast<uint4*>(a.C + static_cast<size_t>(m) * a.ldc + 8 * c) = make_uint4(h[0], h[1], h[2], h[3]);
}

static void launch_splitk_reduce(const GemmArgs& a, hipStream_t s) {
  const long long mn = static_cast<long long>(a.M) * a.N;
  if (a.splits <= 8 && a.N % 8 == 0 && a.ldc % 8 == 0 && aligned16(a.C) && aligned16(a.partial) &&
      mn / 8 < (1LL << 31))
    IRON_LAUNCH(gemm_splitk_reduce8_kernel, dim3(static_cast<unsigned>((mn / 8 + 255) / 256)), dim3(256), 0, s, a);
  else
    IRON_LAUNCH(gemm_splitk_reduce_kernel, dim3(static_cast<unsigned>((mn + 255) / 256)), dim3(256), 0, s, a);
}

// 64x64 tiled transpose through LDS: out (cols, rows) = in (rows, cols)^T.
__global__ __launch_bounds__(256) void transpose_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                        int rows, int cols) {
  __shared__ uint16_t tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int r = e / 64, c = e % 64;
    if (r0 + r < rows && c0 + c < cols) tile[r][c] = in[static_cast<size_t>(r0 + r) * cols + c0 + c];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int c = e / 64, r = e % 64;
    if (r0 + r < rows && c0 + c < cols) out[static_cast<size_t>(c0 + c) * rows + r0 + r] = tile[r][c];
  }
}

}  // namespace
}  // namespace iron

using namespace iron;

static int gemm_check(const char* fn, const void* A, const void* B, const void* C, int M, int N, int K,
                      long long ldc, int epilogue, int has_clamp, float clamp_lo, float clamp_hi) {
  IRON_REQUIRE(A && B && C, "%s: null pointer", fn);
  IRON_REQUIRE(M > 0 && N > 0 && K > 0, "%s: M=%d N=%d K=%d must be positive", fn, M, N, K);
  IRON_REQUIRE(K % BK == 0, "%s: K=%d must be a multiple of %d", fn, K, BK);
  IRON_REQUIRE(K <= kMaxK, "%s: K=%d exceeds %d", fn, K, kMaxK);
  IRON_REQUIRE(aligned16(A) && aligned16(B), "%s: A and B must be 16-byte aligned", fn);
  IRON_REQUIRE(ldc >= N, "%s: ldc=%lld < N=%d", fn, ldc, N);
  const int act = epilogue & ~IRON_EPI_ROUND_TOWARD_ZERO;
  IRON_REQUIRE(act >= EPI_NONE && act <= EPI_GELU_SIGMOID, "%s: bad epilogue %d", fn, epilogue);
  IRON_REQUIRE(!has_clamp || clamp_lo <= clamp_hi, "%s: clamp min > max", fn);
  if ((ldc % 8 == 0) && !aligned16(C)) return fail_einval("%s: C must be 16-byte aligned", fn);
  return 0;
}

template <class T>
static long long tile_count(const GemmArgs& a) {
  return static_cast<long long>((a.M + T::BM - 1) / T::BM) * ((a.N + T::BN - 1) / T::BN) * a.splits;
}

// Cost model: a launch takes ceil(tiles / slots) rounds, each costing a full
// round of tile work at the shape's measured full-occupancy rate (TF/s on one
// MI355X: 256x256 ~1000, 256x192 ~900, 256x128 ~900, 128x128/4 waves ~800, 128x128/8 waves
// ~660). Slots are workgroups resident at once: one per CU, two for the 64 KiB
// shape. Fewer, bigger tiles win on large problems; a problem of one round of
// 128x128 tiles gets the 8-wave shape.
template <class T>
static double launch_cost(const GemmArgs& a, int per_cu, double tflops) {
  const long long slots = 256LL * per_cu, rounds = (tile_count<T>(a) + slots - 1) / slots;
  return static_cast<double>(rounds * slots) * T::BM * T::BN / tflops;
}

template <class T>
static int launch_tile(GemmArgs a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(tile_count<T>(a)));
  if (int rc = take_trace("gemm", grid.x, &a.trace)) return rc;
  if (a.trace)
    IRON_LAUNCH((gemm_nt_kernel<T, true>), grid, dim3(T::kThreads), 0, s, a);
  else
    IRON_LAUNCH((gemm_nt_kernel<T, false>), grid, dim3(T::kThreads), 0, s, a);
  return 0;
}

template <class T>
static void launch_tile_i4(const GemmArgs& a, hipStream_t s) {
  IRON_LAUNCH(gemm_i4_kernel<T>, dim3(static_cast<unsigned>(tile_count<T>(a))), dim3(T::kThreads), 0, s, a);
}

// Shapes whose 128x128 tiles leave CUs idle (with no K split): the smaller
// tile whose count comes closest to one per CU without going over (64 = 64x64,
// 128 = 128x64, 0 = neither fits: the cost model's tiles). 512 tokens, cold
// weights: 512x2048 -> 2048 19.7 -> 12.3 us (64x64), -> 3072 20.0 -> 15.9 us
// (128x64), 512x8192 -> 2048 65.6 -> 40.5 us (64x64).
static int small_tile(int M, int N) {
  auto tiles = [&](int bm, int bn) { return static_cast<long long>((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  if (tiles(128, 128) >= 256) return 0;
  if (tiles(64, 64) <= 256) return 64;
  if (tiles(128, 64) <= 256) return 128;
  return 0;
}

static int gemm_launch(const GemmArgs& a, hipStream_t s) {
  // The SwiGLU pair needs 128-column tiles.
  if (a.splits == 1 && a.epi != kEpiSwigluPair) {
    const int st = small_tile(a.M, a.N);
    if (st == 64) return launch_tile<Tile64>(a, s);
    if (st == 128) return launch_tile<Tile128x64>(a, s);
  }
  const double cl = launch_cost<TileL>(a, 1, 1000.0), cm = launch_cost<TileM>(a, 1, 900.0);
  const double cs = launch_cost<TileS>(a, 1, 660.0), cs2 = launch_cost<TileS2>(a, 2, 800.0);
  // 256x192 only where it divides N exactly (wave quantization: 3968x3072 gets 256 tiles instead of 192 of
  // 256x256; 72 -> 57 us), and never for the SwiGLU pair epilogue, whose 64-column gate/up blocks must pair
  // up inside a tile.
  const double cl3 = (a.N % TileL3::BN == 0 && a.epi != kEpiSwigluPair) ? launch_cost<TileL3>(a, 1, 900.0) : 1e300;
  const double best = std::min(std::min(std::min(cl, cm), std::min(cs, cs2)), cl3);
  if (cl3 == best)
    return launch_tile<TileL3>(a, s);
  else if (cs == best)
    return launch_tile<TileS>(a, s);
  else if (cl == best)
    return launch_tile<TileL>(a, s);
  else if (cm == best)
    return launch_tile<TileM>(a, s);
  else
    return launch_tile<TileS2>(a, s);
}

extern "C" int iron_gemm_bf16_nt(const void* A, const void* B, void* C, int M, int N, int K, long long ldc,
                                 int epilogue, int has_clamp, float clamp_lo, float clamp_hi, void* stream) {
  if (int rc = gemm_check("iron_gemm_bf16_nt", A, B, C, M, N, K, ldc, epilogue, has_clamp, clamp_lo, clamp_hi))
    return rc;
  const long long tiles = static_cast<long long>((M + kSplitTile - 1) / kSplitTile) * ((N + kSplitTile - 1) / kSplitTile);
  IRON_REQUIRE(tiles < (1LL << 31), "iron_gemm_bf16_nt: problem too large");
  GemmArgs a{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), static_cast<uint16_t*>(C), M, N, K,
             ldc, epilogue, has_clamp, clamp_lo, clamp_hi, nullptr, 1};
  set_epilogue(a, epilogue);
  if (int rc = gemm_launch(a, static_cast<hipStream_t>(stream))) return rc;
  return check_launch("gemm_bf16_nt");
}

// Split-K policies, measured (graph replays with cold weights over M =
// 128..2048 for (N, K) = (2048, 2048), (3072, 2048), (2048, 8192), and the
// Llama prefill at 512 tokens).
//
// int4-g32 (iron_gemm_i4g32_nt, whose tiles are 128x128 or larger): split K
// while the workgroups stay within 1.25x the 256 CUs and every range keeps
// >= 8 steps of 64, at most 8 ranges (512x2048->2048: 28.7 us plain, 23.3 in
// 4 ranges; 512x2048->3072: 29.3 plain, 27.4 in 2).
static int splitk_short(int M, int N, int K) {
  const long long tiles = static_cast<long long>((M + kSplitTile - 1) / kSplitTile) * ((N + kSplitTile - 1) / kSplitTile);
  int s = 1;
  while (s < 8 && tiles * s * 2 <= 320 && (K / BK) % (s * 2) == 0 && K / BK / (s * 2) >= 8) s *= 2;
  return s;
}

// Workgroups of the plain bf16 GEMM on a grid that 128x128 tiles leave idle
// (gemm_launch's small_tile), or the 128x128 tile count.
static long long plain_small_grid(int M, int N) {
  const int st = small_tile(M, N);
  const int bm = st == 0 ? 128 : st, bn = st == 0 ? 128 : 64;
  return static_cast<long long>((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

// bf16: a K of fewer than 64 steps is split only when the plain kernel's
// tiles leave CUs idle, and then as the int4 policy does (prefill at 512
// tokens: o_proj, 256 tiles of 64x64, runs unsplit: 12.4 us against 20.5 in
// 4 ranges; qkv, 192 tiles of 128x64, keeps 2 ranges: TTFT 2.05-2.08 ms with
// both split, 2.02-2.05 with neither, 1.99-2.03 so). A long K is split into
// ranges of >= 32 steps, or >= 16 while the workgroups fit one per CU, with
// at most 512 workgroups (K 8192: M 128 and 256 -> 8 ranges, 512 and 1024 ->
// 4, 2048 -> 2; 512x8192->2048: 41.7 us plain, 32.1 in 4).
extern "C" int iron_gemm_splitk_choose(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % BK) return 1;
  if (K / BK < 64) return plain_small_grid(M, N) >= 256 ? 1 : splitk_short(M, N, K);
  const long long tiles = static_cast<long long>((M + kSplitTile - 1) / kSplitTile) * ((N + kSplitTile - 1) / kSplitTile);
  int best = 1;
  for (int s = 2; s <= 8; s *= 2) {
    const int steps = K / BK / s;
    if ((K / BK) % s || tiles * s > 512) break;
    if (steps >= 32 || (steps >= 16 && tiles * s <= 256)) best = s;
  }
  return best;
}

extern "C" int iron_gemm_i4g32_splitk_choose(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % BK) return 1;
  return splitk_short(M, N, K);
}

extern "C" long long iron_gemm_splitk_workspace_bytes(int M, int N, int splits) {
  if (M <= 0 || N <= 0 || splits <= 0) return -1;
  return splits > 1 ? static_cast<long long>(splits) * M * N * 4 : 0;
}

extern "C" int iron_gemm_bf16_nt_splitk(const void* A, const void* B, void* C, int M, int N, int K, long long ldc,
                                        int epilogue, int has_clamp, float clamp_lo, float clamp_hi, int splits,
                                        void* workspace, long long workspace_bytes, void* stream) {
  if (int rc = gemm_check("iron_gemm_bf16_nt_splitk", A, B, C, M, N, K, ldc, epilogue, has_clamp, clamp_lo,
                          clamp_hi))
    return rc;
  IRON_REQUIRE(splits >= 1 && (K / BK) % splits == 0,
               "iron_gemm_bf16_nt_splitk: splits=%d must divide the %d K steps of 64", splits, K / BK);
  if (splits == 1)
    return iron_gemm_bf16_nt(A, B, C, M, N, K, ldc, epilogue, has_clamp, clamp_lo, clamp_hi, stream);
  const long long need = static_cast<long long>(splits) * M * N * 4;
  IRON_REQUIRE(workspace && workspace_bytes >= need, "iron_gemm_bf16_nt_splitk: workspace of %lld bytes < %lld",
               workspace_bytes, need);
  IRON_REQUIRE(aligned16(workspace), "iron_gemm_bf16_nt_splitk: workspace must be 16-byte aligned");
  const long long tiles = static_cast<long long>((M + kSplitTile - 1) / kSplitTile) * ((N + kSplitTile - 1) / kSplitTile) * splits;
  IRON_REQUIRE(tiles < (1LL << 31) && static_cast<long long>(M) * N < (1LL << 38),
               "iron_gemm_bf16_nt_splitk: problem too large");
  GemmArgs a{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), static_cast<uint16_t*>(C), M, N, K,
             ldc, epilogue, has_clamp, clamp_lo, clamp_hi, static_cast<float*>(workspace), splits};
  set_epilogue(a, epilogue);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int rc = gemm_launch(a, s)) return rc;
  launch_splitk_reduce(a, s);
  return check_launch("gemm_bf16_nt_splitk");
}

extern "C" int iron_gemm_bf16_nt_swiglu(const void* A, const void* Bgu, void* H, int M, int F, int K, long long ldh,
                                        void* stream) {
  IRON_REQUIRE(F > 0 && F % 64 == 0, "iron_gemm_bf16_nt_swiglu: F=%d must be a positive multiple of 64", F);
  IRON_REQUIRE(ldh >= F, "iron_gemm_bf16_nt_swiglu: ldh=%lld < F=%d", ldh, F);
  if (int rc = gemm_check("iron_gemm_bf16_nt_swiglu", A, Bgu, H, M, 2 * F, K, 2 * ldh, EPI_NONE, 0, 0.f, 0.f))
    return rc;
  IRON_REQUIRE(ldh % 8 != 0 || aligned16(H), "iron_gemm_bf16_nt_swiglu: H must be 16-byte aligned");
  const long long tiles = static_cast<long long>((M + kSplitTile - 1) / kSplitTile) * ((2 * F) / kSplitTile);
  IRON_REQUIRE(tiles < (1LL << 31), "iron_gemm_bf16_nt_swiglu: problem too large");
  GemmArgs a{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(Bgu), static_cast<uint16_t*>(H), M, 2 * F,
             K, ldh, kEpiSwigluPair, 0, 0.f, 0.f, nullptr, 1};
  if (int rc = gemm_launch(a, static_cast<hipStream_t>(stream))) return rc;
  return check_launch("gemm_bf16_nt_swiglu");
}

// Cost model for the int4 kernels (measured full-occupancy rates, TFLOP/s).
static void gemm_i4_launch(const GemmArgs& a, hipStream_t s) {
  const double cs = launch_cost<TileI4S>(a, 1, 600.0), cm = launch_cost<TileI4M>(a, 1, 800.0);
  if (cs <= cm)
    launch_tile_i4<TileI4S>(a, s);
  else
    launch_tile_i4<TileI4M>(a, s);
}

extern "C" int iron_gemm_i4g32_nt(const void* A, const void* codes, const void* scales, void* C, int M, int N, int K,
                                  long long ldc, int epilogue, int has_clamp, float clamp_lo, float clamp_hi,
                                  int is_signed, int splits, void* workspace, long long workspace_bytes,
                                  void* stream) {
  if (int rc = gemm_check("iron_gemm_i4g32_nt", A, codes, C, M, N, K, ldc, epilogue, has_clamp, clamp_lo, clamp_hi))
    return rc;
  IRON_REQUIRE(scales && (reinterpret_cast<uintptr_t>(scales) & 3u) == 0,
               "iron_gemm_i4g32_nt: scales must be non-null and 4-byte aligned");
  IRON_REQUIRE(splits >= 1 && (K / BK) % splits == 0,
               "iron_gemm_i4g32_nt: splits=%d must divide the %d K steps of 64", splits, K / BK);
  const long long tiles =
      static_cast<long long>((M + kSplitTile - 1) / kSplitTile) * ((N + kSplitTile - 1) / kSplitTile) * splits;
  IRON_REQUIRE(tiles < (1LL << 31) && static_cast<long long>(M) * N < (1LL << 38),
               "iron_gemm_i4g32_nt: problem too large");
  float* partial = nullptr;
  if (splits > 1) {
    const long long need = static_cast<long long>(splits) * M * N * 4;
    IRON_REQUIRE(workspace && workspace_bytes >= need, "iron_gemm_i4g32_nt: workspace of %lld bytes < %lld",
                 workspace_bytes, need);
    IRON_REQUIRE(aligned16(workspace), "iron_gemm_i4g32_nt: workspace must be 16-byte aligned");
    partial = static_cast<float*>(workspace);
  }
  GemmArgs a{static_cast<const uint16_t*>(A), nullptr, static_cast<uint16_t*>(C), M, N, K, ldc, epilogue, has_clamp,
             clamp_lo, clamp_hi, partial, splits, static_cast<const uint8_t*>(codes),
             static_cast<const uint16_t*>(scales), is_signed ? 1 : 0};
  set_epilogue(a, epilogue);
  hipStream_t s = static_cast<hipStream_t>(stream);
  gemm_i4_launch(a, s);
  if (splits > 1) launch_splitk_reduce(a, s);
  return check_launch("gemm_i4g32_nt");
}

extern "C" int iron_gemm_nt_partials(const void* A, const void* B, const void* codes, const void* scales,
                                     int is_signed, int M, int N, int K, int splits, void* workspace,
                                     long long workspace_bytes, void* stream) {
  const bool i4 = codes != nullptr;
  IRON_REQUIRE(i4 != (B != nullptr), "iron_gemm_nt_partials: give exactly one of B (bf16) and codes (int4-g32)");
  if (int rc = gemm_check("iron_gemm_nt_partials", A, i4 ? codes : B, workspace, M, N, K, N, EPI_NONE, 0, 0.f, 0.f))
    return rc;
  IRON_REQUIRE(!i4 || (scales && (reinterpret_cast<uintptr_t>(scales) & 3u) == 0),
               "iron_gemm_nt_partials: scales must be non-null and 4-byte aligned");
  IRON_REQUIRE(splits >= 1 && (K / BK) % splits == 0,
               "iron_gemm_nt_partials: splits=%d must divide the %d K steps of 64", splits, K / BK);
  const long long tiles =
      static_cast<long long>((M + kSplitTile - 1) / kSplitTile) * ((N + kSplitTile - 1) / kSplitTile) * splits;
  const long long need = static_cast<long long>(splits) * M * N * 4;
  IRON_REQUIRE(tiles < (1LL << 31) && static_cast<long long>(M) * N < (1LL << 38),
               "iron_gemm_nt_partials: problem too large");
  IRON_REQUIRE(workspace_bytes >= need, "iron_gemm_nt_partials: workspace of %lld bytes < %lld", workspace_bytes,
               need);
  IRON_REQUIRE(aligned16(workspace), "iron_gemm_nt_partials: workspace must be 16-byte aligned");
  GemmArgs a{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), nullptr, M, N, K, N, EPI_NONE, 0,
             0.f, 0.f, static_cast<float*>(workspace), splits, static_cast<const uint8_t*>(codes),
             static_cast<const uint16_t*>(scales), is_signed ? 1 : 0};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (i4)
    gemm_i4_launch(a, s);
  else if (int rc = gemm_launch(a, s))
    return rc;
  return check_launch("gemm_nt_partials");
}

extern "C" int iron_transpose_bf16(const void* in, void* out, int rows, int cols, void* stream) {
  IRON_REQUIRE(in && out && in != out, "iron_transpose_bf16: null or aliased pointers");
  IRON_REQUIRE(rows > 0 && cols > 0, "iron_transpose_bf16: empty matrix");
  dim3 grid((cols + 63) / 64, (rows + 63) / 64);
  IRON_REQUIRE(grid.y < 65536, "iron_transpose_bf16: too many rows");
  IRON_LAUNCH(transpose_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), rows, cols);
  return check_launch("transpose_bf16");
}
