// Matrix-vector kernels for batch-1 decode: bf16 GEMV, fused int4-group-32
// GEMV and the int4 dequantizers.
//
// All of them stream the weight matrix from HBM exactly once with 16-byte
// nontemporal loads. One wavefront owns one (bf16) or R (int4) output rows;
// each lane walks the row in 16-byte chunks strided by 64 chunks, so one load
// instruction moves a contiguous 1 KiB per wave. Products accumulate in fp32
// (v_dot2c_f32_bf16) and the row total is a DPP wave reduction.
//
// Each kernel has a fast path, specialised at compile time for the shapes of
// the Llama decode step (every load issued up front, no bounds checks in the
// unrolled body), and a generic path for any other valid shape.
//
// Optional fusions (used by the decode step, all off for the plain operator):
//   norm_w   : the input vector is RMS-normalised and scaled by norm_w first
//              (every wave recomputes sum(x^2); x is a few KiB and L2-resident)
//   W2       : a second matrix of the same shape; the output is
//              silu(W.x) * (W2.x)   (the SwiGLU gate/up pair)
//   residual : added to the (activated) result before the bf16 rounding
#include <type_traits>

#include "iron_common.hpp"
#include "i4_dot.hpp"
#include "trace.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

// norm_mode: what the optional RMSNorm does to the input vector x.
//   NORM_NONE   : x used as given
//   NORM_WEIGHT : x -> bf16(x * rsqrt(mean(x^2) + eps) * norm_w)  (reference order)
//   NORM_SCALE  : outputs scaled by rsqrt(mean(x^2) + eps); the norm weight is
//                 folded into the matrix columns beforehand, so no per-element
//                 normalisation is needed (what the decode step uses)
enum NormMode : int { NORM_NONE = 0, NORM_WEIGHT = 1, NORM_SCALE = 2 };

struct GemvArgs {
  const uint16_t* W;       // (batches, M, K) bf16
  const uint16_t* W2;      // optional second (M, K) matrix (SwiGLU up projection)
  const uint16_t* x;       // (batches, K) bf16
  uint16_t* y;             // (batches, M) bf16
  const uint16_t* norm_w;  // (K,) RMSNorm weight for NORM_WEIGHT
  const uint16_t* resid;   // optional (M,) residual
  unsigned long long* keys;  // optional argmax key per workgroup (4 rows)
  int M, K;
  float eps;
  int epi;
  unsigned* epoch;  // optional: advanced by one (skipping 0) by the first thread of the grid
};

__device__ __forceinline__ float dot_chunk(uint4 w, uint4 x, float acc) {
  acc = dot2_bf16(w.x, x.x, acc);
  acc = dot2_bf16(w.y, x.y, acc);
  acc = dot2_bf16(w.z, x.z, acc);
  acc = dot2_bf16(w.w, x.w, acc);
  return acc;
}

// inv_rms of a K-vector (K % 8 == 0), computed by one wave (all lanes get it).
__device__ __forceinline__ float wave_inv_rms(const uint16_t* x, int K, float eps, int lane) {
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  float ss = 0.f;
  for (int c = lane; c < (K >> 3); c += kWave) ss = sumsq_chunk(xv[c], ss);
  ss = wave_sum(ss);
  return inv_rms(ss, K, eps);
}

// Final value of one output row (activation or SwiGLU, residual), stored as
// bf16; returns the stored value for the argmax keys.
// `rv` is the row's residual (already loaded; used only when has_resid).
__device__ __forceinline__ float finish_row(bool has_resid, float rv, int epi, uint16_t* y, size_t idx, float acc,
                                            float acc2, bool pair) {
  float v = pair ? silu_f32(acc) * acc2 : apply_epilogue(acc, epi);
  if (has_resid) v += rv;
  const uint16_t o = f32_to_bf16(v);
  y[idx] = o;
  return bf16_to_f32(o);
}

// Workgroup argmax of the rows its waves produced, one key per 4 rows: with R
// rows per wave, waves 4/R*g .. 4/R*g + 4/R - 1 form key g of the workgroup,
// written to keys[key_idx * R + g] when that index is below n_keys.
// Every wave of the workgroup must call it (inactive waves pass key 0).
template <int R = 1>
__device__ __forceinline__ void publish_key(unsigned long long* keys, size_t key_idx, unsigned long long key,
                                            size_t n_keys = ~size_t(0)) {
  static_assert(R == 1 || R == 2 || R == 4, "4 rows per key");
  constexpr int WPK = 4 / R;  // waves per key
  __shared__ unsigned long long ks[4];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & (kWave - 1)) == 0) ks[wave] = key;
  __syncthreads();
  if (threadIdx.x < R) {
    const int g = threadIdx.x;
    unsigned long long b = ks[g * WPK];
    for (int w = 1; w < WPK; ++w) b = ks[g * WPK + w] > b ? ks[g * WPK + w] : b;
    const size_t idx = key_idx * R + g;
    if (idx < n_keys) keys[idx] = b;
  }
}

// The epoch word of the one-launch decode step (its exchange tags) moves on
// once per step; the head GEMV that ends the step does it, after every
// workgroup of the step's launch has read the old value. Only launches with
// argmax keys pass an epoch: every thread of workgroup 0 reaches the end.
__device__ __forceinline__ void advance_epoch(unsigned* epoch) {
  if (epoch && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    const unsigned e = *epoch + 1u;
    *epoch = e ? e : 1u;
  }
}

// Fast path: K == 512*U exactly; each lane holds U chunks of W (and W2) in
// flight. One wave per output row.
// W, W2, x, the residual and M come as leading arguments, preloaded into SGPRs
// by the dispatch (as for the int4 fast path), and K is 512 U; an inactive
// wave does not leave early, since that test would wait for the keys argument.
template <int U, bool PAIR, int NM>
__global__ __launch_bounds__(256) void gemv_bf16_fast(const uint16_t* W, const uint16_t* W2, const uint16_t* xin,
                                                     const uint16_t* resid, int M, GemvArgs a) {
  constexpr int K = 512 * U;
  const int lane = threadIdx.x & (kWave - 1);
  const int tile = blockIdx.x;  // round-robin rows (see iron_gemv_bf16)
  const int row = tile * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  const bool active = row < M;  // uniform per wave
  unsigned long long key = 0;
  if (active) {
    const uint16_t* x = xin + static_cast<size_t>(b) * K;
    const size_t roff = (static_cast<size_t>(b) * M + row) * static_cast<size_t>(K);
    const uint4* Wr = reinterpret_cast<const uint4*>(W + roff) + lane;
    const uint4* W2r = PAIR ? reinterpret_cast<const uint4*>(W2 + roff) + lane : nullptr;
    const uint4* xv = reinterpret_cast<const uint4*>(x) + lane;

    uint4 w[U], w2[U], xc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      w[u] = ld_stream16(Wr + u * kWave);
      if (PAIR) w2[u] = ld_stream16(W2r + u * kWave);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) xc[u] = xv[u * kWave];
    // The residual is loaded with the operands, not after the reduction; the
    // load is unconditional (x[0] stands in when there is none) so that no
    // branch makes the compiler wait for every load in flight.
    const float rv = bf16_to_f32(resid ? resid[row] : xin[0]);
    float inv = 1.f;
    if (NM != NORM_NONE) {
      float ss = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) ss = sumsq_chunk(xc[u], ss);
      inv = inv_rms(wave_sum(ss), K, a.eps);
    }
    if (NM == NORM_WEIGHT) {
      const uint4* nw = reinterpret_cast<const uint4*>(a.norm_w) + lane;
#pragma unroll
      for (int u = 0; u < U; ++u) xc[u] = normalize_chunk(xc[u], nw[u * kWave], inv);
    }
    float acc = 0.f, acc2 = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc = dot_chunk(w[u], xc[u], acc);
      if (PAIR) acc2 = dot_chunk(w2[u], xc[u], acc2);
    }
    acc = wave_sum(acc);
    if (PAIR) acc2 = wave_sum(acc2);
    if (NM == NORM_SCALE) {
      acc *= inv;
      acc2 *= inv;
    }
    float v = 0.f;
    if (lane == 0) v = finish_row(resid != nullptr, rv, a.epi, a.y, static_cast<size_t>(b) * M + row, acc, acc2, PAIR);
    if (a.keys) key = argmax_key(__shfl(v, 0, kWave), row);
  }
  if (a.keys) publish_key(a.keys, static_cast<size_t>(b) * gridDim.x + tile, key);
  advance_epoch(a.epoch);  // last: at the start it would serialise the argument loads
}

// Generic path: any K % 8 == 0; chunks streamed 4 per lane per iteration.
template <bool PAIR>
__global__ __launch_bounds__(256) void gemv_bf16_generic(GemvArgs a, int norm_mode) {
  const int lane = threadIdx.x & (kWave - 1);
  const int tile = blockIdx.x;
  const int row = tile * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  const bool active = row < a.M;
  if (!active && !a.keys) return;
  unsigned long long key = 0;
  if (active) {
    constexpr int U = 4;
    const int nch = a.K >> 3;
    const uint16_t* x = a.x + static_cast<size_t>(b) * a.K;
    const uint4* xv = reinterpret_cast<const uint4*>(x);
    const uint4* nw = reinterpret_cast<const uint4*>(a.norm_w);
    const float inv = norm_mode != NORM_NONE ? wave_inv_rms(x, a.K, a.eps, lane) : 1.f;
    const size_t roff = (static_cast<size_t>(b) * a.M + row) * static_cast<size_t>(a.K);
    const uint4* Wr = reinterpret_cast<const uint4*>(a.W + roff);
    const uint4* W2r = PAIR ? reinterpret_cast<const uint4*>(a.W2 + roff) : nullptr;
    float acc = 0.f, acc2 = 0.f;
    for (int base = lane; base < nch; base += kWave * U) {
      uint4 w[U], w2[U], xc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = base + u * kWave;
        const bool ok = c < nch;
        w[u] = ok ? ld_stream16(Wr + c) : make_uint4(0, 0, 0, 0);
        if (PAIR) w2[u] = ok ? ld_stream16(W2r + c) : make_uint4(0, 0, 0, 0);
        xc[u] = ok ? xv[c] : make_uint4(0, 0, 0, 0);
        if (ok && norm_mode == NORM_WEIGHT) xc[u] = normalize_chunk(xc[u], nw[c], inv);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        acc = dot_chunk(w[u], xc[u], acc);
        if (PAIR) acc2 = dot_chunk(w2[u], xc[u], acc2);
      }
    }
    acc = wave_sum(acc);
    if (PAIR) acc2 = wave_sum(acc2);
    if (norm_mode == NORM_SCALE) {
      acc *= inv;
      acc2 *= inv;
    }
    float v = 0.f;
    if (lane == 0) {
      const float rv = a.resid ? bf16_to_f32(a.resid[row]) : 0.f;
      v = finish_row(a.resid != nullptr, rv, a.epi, a.y, static_cast<size_t>(b) * a.M + row, acc, acc2, PAIR);
    }
    if (a.keys) key = argmax_key(__shfl(v, 0, kWave), row);
  }
  if (a.keys) publish_key(a.keys, static_cast<size_t>(b) * gridDim.x + tile, key);
  advance_epoch(a.epoch);  // last: at the start it would serialise the argument loads
}

template <int U, bool PAIR>
void launch_bf16_fast(const GemvArgs& a, int norm_mode, dim3 grid, hipStream_t s) {
#define IRON_BF16_FAST(NM) \
  IRON_LAUNCH((gemv_bf16_fast<U, PAIR, NM>), grid, dim3(256), 0, s, a.W, a.W2, a.x, a.resid, a.M, a)
  switch (norm_mode) {
    case NORM_WEIGHT: IRON_BF16_FAST(NORM_WEIGHT); break;
    case NORM_SCALE: IRON_BF16_FAST(NORM_SCALE); break;
    default: IRON_BF16_FAST(NORM_NONE); break;
  }
#undef IRON_BF16_FAST
}

template <bool PAIR>
int launch_gemv_bf16(const GemvArgs& a, int norm_mode, int batches, hipStream_t s) {
  dim3 grid((a.M + 3) / 4, batches);
  const int U = (a.K % 512 == 0) ? a.K / 512 : 0;
  switch (U) {
    case 1: launch_bf16_fast<1, PAIR>(a, norm_mode, grid, s); break;
    case 2: launch_bf16_fast<2, PAIR>(a, norm_mode, grid, s); break;
    case 4: launch_bf16_fast<4, PAIR>(a, norm_mode, grid, s); break;
    case 8: launch_bf16_fast<8, PAIR>(a, norm_mode, grid, s); break;
    case 16:
      if (!PAIR) {
        launch_bf16_fast<16, false>(a, norm_mode, grid, s);
        break;
      }
      [[fallthrough]];
    default: IRON_LAUNCH((gemv_bf16_generic<PAIR>), grid, dim3(256), 0, s, a, norm_mode); break;
  }
  return check_launch("gemv_bf16");
}

// ---------------------------------------------------------------------------
// int4, group 32. codes (M, K/2) uint8, two weights per byte along K, low
// nibble first; scales (M, K/32) bf16. One 16-byte chunk of codes is exactly
// one group, so lane l owns groups l, l+64, ... of every row it touches. The
// group inner products are dequant-free (i4_dot.hpp).
// ---------------------------------------------------------------------------
struct I4Args {
  const uint8_t* codes;
  const uint16_t* scales;
  const uint8_t* codes2;  // optional SwiGLU up projection
  const uint16_t* scales2;
  const uint16_t* x;
  uint16_t* y;
  const uint16_t* norm_w;
  const uint16_t* resid;
  unsigned long long* keys;  // optional argmax key per 4 rows (R rows per wave: R keys per workgroup)
  int M, K;
  float eps;
  int epi;
  uint32_t magic;  // 0x43084308 signed two's-complement nibbles, 0x43004300 unsigned
  float offset;    // 136 signed, 128 unsigned
  unsigned* epoch;  // optional: advanced by one (skipping 0) by the first thread of the grid
  void* trace;      // phase trace records (trace.hpp), or null
};

// Fast path: K == 2048*GPL*KS. The 4 waves of a workgroup form 4/KS row
// groups of R rows; the KS waves of a row group split K, each lane owning GPL
// groups of 32 per row, and their partial sums meet in LDS. R rows of one
// wave share the x preparation.
// TR: the instance launched while a phase trace is armed (trace.hpp); the
// others carry no trace code, whose clock read at entry measured 0.1 us of the
// headline launch.
// The pointers and the row count that the first loads need come as leading
// arguments, which the dispatch preloads into SGPRs (the kernarg preload
// count of this file's build); the rest of I4Args is read from the kernel
// argument segment while those loads are in flight. With every argument in the
// struct, no wave could issue a load before its argument fetch returned: the
// headline 8192 x 2048 launch took 3.97 us that way against 3.42 with the
// leading arguments preloaded (same outputs). Rows are XCD-contiguous
// (xcd_tile; measured faster for every int4 shape of the decode step), and for
// the same reason the grid size behind that order comes from M, not from the
// dispatch packet.
template <int GPL, int R, int KS, bool PAIR, int NM, bool TR>
__global__ __launch_bounds__(256) void gemv_i4_fast(const uint8_t* codes, const uint16_t* scales, const uint16_t* x,
                                                   const uint8_t* codes2, const uint16_t* scales2,
                                                   const uint16_t* resid, int M, I4Args a) {
  static_assert(KS == 1 || KS == 2 || KS == 4, "KS divides the 4 waves");
  constexpr int kRowsPerBlock = R * 4 / KS;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  // trace points: 0 start, 1 x prepared, 2 row products done
  void* const trace = TR ? a.trace : nullptr;
  unsigned long long t_start = 0;
  if constexpr (TR) t_start = trace_clock();
  const int tile = xcd_tile((M + kRowsPerBlock - 1) / kRowsPerBlock);
  const int rg = wave / KS, kp = wave % KS;
  const int row0 = (tile * (4 / KS) + rg) * R;
  // uniform per row group; an inactive wave does not leave early, since that
  // test would wait for the keys argument before the first load is issued
  const bool active = row0 < M;
  constexpr int G = GPL * kWave * KS;                   // groups per row
  constexpr size_t crow = static_cast<size_t>(G) * 16;  // code bytes per row
  const int g0 = kp * GPL * kWave + lane;               // this lane's first group
  float part[R][2], rres[R];
  float inv = 1.f, ss = 0.f;
  if (active) {
    // x and the norm weight first (L2 hits shared by every wave), then the
    // weight rows, their scales and the residuals, all issued before the first
    // wait: x is prepared while the weights are in flight. The fence keeps the
    // scheduler from sinking the later rows' scale or code loads below the
    // first row's products, which added a dependent HBM round trip to every
    // wave (measured: SwiGLU pair 4-7% and o_proj 4% faster with it). Issuing
    // x after the weights instead was 7-11% slower.
    uint4 xr[GPL][4];
    const uint4* xv = reinterpret_cast<const uint4*>(x);
#pragma unroll
    for (int j = 0; j < GPL; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) xr[j][q] = xv[(g0 + j * kWave) * 4 + q];
    uint4 nwr[GPL][4];
    if (NM == NORM_WEIGHT) {
      const uint4* nw = reinterpret_cast<const uint4*>(a.norm_w);
#pragma unroll
      for (int j = 0; j < GPL; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) nwr[j][q] = nw[(g0 + j * kWave) * 4 + q];
    }
    uint4 cw[R][GPL], cw2[R][GPL];
    uint16_t sc[R][GPL], sc2[R][GPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const size_t row = static_cast<size_t>(row0 + r);
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        const int g = g0 + j * kWave;
        cw[r][j] = ld_stream16(codes + row * crow + static_cast<size_t>(g) * 16);
        if (PAIR) cw2[r][j] = ld_stream16(codes2 + row * crow + static_cast<size_t>(g) * 16);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const size_t row = static_cast<size_t>(row0 + r);
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        const int g = g0 + j * kWave;
        sc[r][j] = scales[row * G + g];
        if (PAIR) sc2[r][j] = scales2[row * G + g];
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) rres[r] = bf16_to_f32(resid ? resid[row0 + r] : x[0]);  // unconditional load
    __builtin_amdgcn_sched_barrier(0);
    trace_write(trace, kTraceGemvI4, blockIdx.x, 0, t_start);
    if (NM != NORM_NONE) {
#pragma unroll
      for (int j = 0; j < GPL; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) ss = sumsq_chunk(xr[j][q], ss);
      ss = wave_sum(ss);
      if (KS == 1) inv = inv_rms(ss, a.K, a.eps);
    }
    if (NM == NORM_WEIGHT) {
      if (KS > 1) {  // the full sum of squares is needed before the products
        __shared__ float ss_s[4];
        if (lane == 0) ss_s[wave] = ss;
        __syncthreads();
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < KS; ++k) t += ss_s[rg * KS + k];
        inv = inv_rms(t, a.K, a.eps);
      }
#pragma unroll
      for (int j = 0; j < GPL; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) xr[j][q] = normalize_chunk(xr[j][q], nwr[j][q], inv);
    }
    XGroup xg[GPL];
#pragma unroll
    for (int j = 0; j < GPL; ++j) build_xgroup(xr[j], xg[j]);
    // x is prepared while the weights are still in flight: without this fence
    // the compiler hoisted the scale conversions above it, and its wait for
    // them (counts are in issue order) also waited for every code load.
    __builtin_amdgcn_sched_barrier(0);
    trace_stamp(trace, kTraceGemvI4, blockIdx.x, 1);

#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc = 0.f, acc2 = 0.f;
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        const float d = i4_group_total(cw[r][j], xg[j], a.magic, a.offset);
        acc = fmaf(bf16_to_f32(sc[r][j]), d, acc);
        if (PAIR) {
          const float d2 = i4_group_total(cw2[r][j], xg[j], a.magic, a.offset);
          acc2 = fmaf(bf16_to_f32(sc2[r][j]), d2, acc2);
        }
      }
      part[r][0] = wave_sum(acc);
      part[r][1] = PAIR ? wave_sum(acc2) : 0.f;
    }
    trace_stamp(trace, kTraceGemvI4, blockIdx.x, 2);
  }
  if (KS > 1) {  // K-split partners meet in LDS; the kp == 0 wave finishes the rows
    __shared__ float p_s[4][R][2];
    __shared__ float q_s[4];
    if (lane == 0 && active) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        p_s[wave][r][0] = part[r][0];
        p_s[wave][r][1] = part[r][1];
      }
      q_s[wave] = ss;
    }
    __syncthreads();
    if (kp != 0 || !active) return;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int k = 1; k < KS; ++k) {
        part[r][0] += p_s[wave + k][r][0];
        part[r][1] += p_s[wave + k][r][1];
      }
    if (NM == NORM_SCALE) {
      float t = ss;
#pragma unroll
      for (int k = 1; k < KS; ++k) t += q_s[wave + k];
      inv = inv_rms(t, a.K, a.eps);
    }
  }
  unsigned long long key = 0;
  if (active) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float t = part[r][0], t2 = part[r][1];
      if (NM == NORM_SCALE) {
        t *= inv;
        t2 *= inv;
      }
      float v = 0.f;
      if (lane == 0) v = finish_row(resid != nullptr, rres[r], a.epi, a.y, row0 + r, t, t2, PAIR);
      if (KS == 1 && a.keys) {
        const unsigned long long k = argmax_key(__shfl(v, 0, kWave), row0 + r);
        key = k > key ? k : key;
      }
    }
  }
  if (KS == 1 && a.keys) publish_key<R>(a.keys, tile, key, (static_cast<size_t>(M) + 3) / 4);
  advance_epoch(a.epoch);  // last: at the start it would serialise the argument loads
}

// Generic path: any K % 32 == 0, one row per wave, groups streamed one at a time.
template <bool PAIR>
__global__ __launch_bounds__(256) void gemv_i4_generic(I4Args a, int norm_mode) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool active = row < a.M;
  if (!active && !a.keys) return;
  unsigned long long key = 0;
  if (active) {
    const int G = a.K >> 5;
    const size_t crow = static_cast<size_t>(a.K) >> 1;
    const uint4* xv = reinterpret_cast<const uint4*>(a.x);
    const uint4* nw = reinterpret_cast<const uint4*>(a.norm_w);
    const float inv = norm_mode != NORM_NONE ? wave_inv_rms(a.x, a.K, a.eps, lane) : 1.f;
    float acc = 0.f, acc2 = 0.f;
    for (int g = lane; g < G; g += kWave) {
      const uint4 c = ld_stream16(a.codes + row * crow + static_cast<size_t>(g) * 16);
      const float s = bf16_to_f32(a.scales[static_cast<size_t>(row) * G + g]);
      uint4 c2 = make_uint4(0, 0, 0, 0);
      float s2 = 0.f;
      if (PAIR) {
        c2 = ld_stream16(a.codes2 + row * crow + static_cast<size_t>(g) * 16);
        s2 = bf16_to_f32(a.scales2[static_cast<size_t>(row) * G + g]);
      }
      uint4 xc[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xc[q] = xv[g * 4 + q];
        if (norm_mode == NORM_WEIGHT) xc[q] = normalize_chunk(xc[q], nw[g * 4 + q], inv);
      }
      XGroup t;
      build_xgroup(xc, t);
      acc = fmaf(s, i4_group_total(c, t, a.magic, a.offset), acc);
      if (PAIR) acc2 = fmaf(s2, i4_group_total(c2, t, a.magic, a.offset), acc2);
    }
    float t = wave_sum(acc);
    float t2 = PAIR ? wave_sum(acc2) : 0.f;
    if (norm_mode == NORM_SCALE) {
      t *= inv;
      t2 *= inv;
    }
    float v = 0.f;
    if (lane == 0) {
      const float rv = a.resid ? bf16_to_f32(a.resid[row]) : 0.f;
      v = finish_row(a.resid != nullptr, rv, a.epi, a.y, row, t, t2, PAIR);
    }
    if (a.keys) key = argmax_key(__shfl(v, 0, kWave), row);
  }
  if (a.keys) publish_key(a.keys, blockIdx.x, key);
  advance_epoch(a.epoch);
}

template <int GPL, int R, int KS, bool PAIR>
int launch_i4_fast(I4Args a, int norm_mode, hipStream_t s) {
  const int rows_per_block = R * 4 / KS;
  dim3 grid((a.M + rows_per_block - 1) / rows_per_block), block(256);
  if (int rc = take_trace("iron_gemv_i4g32", grid.x, &a.trace)) return rc;
  auto go = [&](auto tr) {
    constexpr bool TR = decltype(tr)::value;
#define IRON_I4_FAST(NM)                                                                                       \
  IRON_LAUNCH((gemv_i4_fast<GPL, R, KS, PAIR, NM, TR>), grid, block, 0, s, a.codes, a.scales, a.x, a.codes2, \
              a.scales2, a.resid, a.M, a)
    switch (norm_mode) {
      case NORM_WEIGHT: IRON_I4_FAST(NORM_WEIGHT); break;
      case NORM_SCALE: IRON_I4_FAST(NORM_SCALE); break;
      default: IRON_I4_FAST(NORM_NONE); break;
    }
#undef IRON_I4_FAST
  };
  if (a.trace)
    go(std::true_type{});
  else
    go(std::false_type{});
  return 0;
}

template <bool PAIR>
int launch_gemv_i4(const I4Args& a, int norm_mode, hipStream_t s) {
  // Argmax keys are defined per 4 rows: no K split, and R rows per wave give R
  // keys per workgroup. Very long matrices (the lm_head) take 4 rows per wave:
  // they run many rounds of waves, each paying the load latency, so more bytes
  // in flight per wave pay (128256x2048: 1 row per wave 46 us, 2 rows 33 us,
  // 4 rows 27.5 us); at 8192 rows 4 per wave was 6% slower than 2.
  int rc = 0;  // a refused trace request (take_trace)
  if (a.keys) {
    if (a.K == 2048 && a.M % 4 == 0 && a.M >= 65536) rc = launch_i4_fast<1, 4, 1, PAIR>(a, norm_mode, s);
    else if (a.K == 2048 && a.M % 2 == 0 && a.M >= 8192) rc = launch_i4_fast<1, 2, 1, PAIR>(a, norm_mode, s);
    else if (a.K == 2048) rc = launch_i4_fast<1, 1, 1, PAIR>(a, norm_mode, s);
    else IRON_LAUNCH((gemv_i4_generic<PAIR>), dim3((a.M + 3) / 4), dim3(256), 0, s, a, norm_mode);
    return rc ? rc : check_launch("gemv_i4g32");
  }
  // Two rows per wave share x when there are enough rows to keep >= 4 waves
  // per SIMD (for the SwiGLU pair, two rows of each matrix); longer rows are
  // split over 2 or 4 waves.
  const bool r2 = a.M % 2 == 0 && a.M >= 8192;
  switch (a.K) {
    case 2048:
      if (!PAIR && a.M % 4 == 0 && a.M >= 65536) {  // the lm_head shape: 31.3 -> 25.6 us
        rc = launch_i4_fast<1, 4, 1, PAIR>(a, norm_mode, s);
        break;
      }
      if (r2) rc = launch_i4_fast<1, 2, 1, PAIR>(a, norm_mode, s);
      else rc = launch_i4_fast<1, 1, 1, PAIR>(a, norm_mode, s);
      break;
    case 4096:  // a workgroup is 2 row groups: both must be inside M
      if (a.M % 2 == 0) {
        rc = launch_i4_fast<1, 1, 2, PAIR>(a, norm_mode, s);
        break;
      }
      [[fallthrough]];
    case 8192:
      if (a.K == 8192) {
        // One wave per row pair, four groups per lane (2048x8192 + residual with cold weights: 4.56 us,
        // against 4.69 with four waves splitting each row and 5.2 with two); the SwiGLU pair keeps four
        // waves per row.
        if (!PAIR && a.M % 2 == 0) rc = launch_i4_fast<4, 2, 1, PAIR>(a, norm_mode, s);
        else rc = launch_i4_fast<1, 1, 4, PAIR>(a, norm_mode, s);
        break;
      }
      [[fallthrough]];
    default:
      IRON_LAUNCH((gemv_i4_generic<PAIR>), dim3((a.M + 3) / 4), dim3(256), 0, s, a, norm_mode);
      break;
  }
  return rc ? rc : check_launch("gemv_i4g32");
}

// ---------------------------------------------------------------------------
// Dequantizers (bit-exact: bf16_rne(float(q) * float(scale))).
// ---------------------------------------------------------------------------

// Planar: codes (N, K/2), scales (N, K/group). One thread = 8 consecutive
// weights (4 code bytes -> one 16-byte store).
__global__ __launch_bounds__(256) void dequant_planar_kernel(const uint8_t* __restrict__ codes,
                                                             const uint16_t* __restrict__ scales,
                                                             uint16_t* __restrict__ out, int N, int K,
                                                             int group, int is_signed) {
  const size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t per_row = static_cast<size_t>(K) >> 3;
  if (t >= per_row * static_cast<size_t>(N)) return;
  const size_t row = t / per_row;
  const int k0 = static_cast<int>(t - row * per_row) * 8;
  const uint32_t w = *reinterpret_cast<const uint32_t*>(codes + row * (K >> 1) + (k0 >> 1));
  const int G = K / group;
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int n = (w >> (4 * (e + h))) & 0xf;
      const int q = is_signed ? ((n ^ 8) - 8) : n;
      const float s = bf16_to_f32(scales[row * G + (k0 + e + h) / group]);
      v[h] = static_cast<float>(q) * s;
    }
    o[e >> 1] = pack_bf16x2(v[0], v[1]);
  }
  *reinterpret_cast<uint4*>(out + row * K + k0) = make_uint4(o[0], o[1], o[2], o[3]);
}

// Tile payload: per tile, tile/2 code bytes then tile/group bf16 scales
// (little-endian bytes). One thread = 2 weights (one code byte).
__global__ __launch_bounds__(256) void dequant_payload_kernel(const uint8_t* __restrict__ payload,
                                                              uint16_t* __restrict__ out, long long size,
                                                              int tile, int group, int is_signed) {
  const long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  const long long e0 = t * 2;
  if (e0 >= size) return;
  const long long tile_idx = e0 / tile;
  const int in_tile = static_cast<int>(e0 - tile_idx * tile);
  const long long tile_bytes = tile / 2 + 2LL * (tile / group);
  const uint8_t* base = payload + tile_idx * tile_bytes;
  const uint8_t byte = base[in_tile >> 1];
  const int sidx = in_tile / group;  // both weights of a byte share a group (group is even)
  const uint8_t* sp = base + tile / 2 + 2 * sidx;
  const float s = bf16_to_f32(static_cast<uint16_t>(sp[0] | (sp[1] << 8)));
  const int n0 = byte & 0xf, n1 = byte >> 4;
  const int q0 = is_signed ? ((n0 ^ 8) - 8) : n0;
  const int q1 = is_signed ? ((n1 ^ 8) - 8) : n1;
  out[e0] = f32_to_bf16(static_cast<float>(q0) * s);
  out[e0 + 1] = f32_to_bf16(static_cast<float>(q1) * s);
}

}  // namespace
}  // namespace iron

using namespace iron;

extern "C" int iron_gemv_bf16(const void* W, const void* x, void* y, int M, int K, int batches,
                              int epilogue, void* stream) {
  IRON_REQUIRE(W && x && y, "iron_gemv_bf16: null pointer");
  IRON_REQUIRE(M > 0 && K > 0 && batches > 0, "iron_gemv_bf16: M=%d K=%d batches=%d must be positive", M,
               K, batches);
  IRON_REQUIRE(K % 8 == 0, "iron_gemv_bf16: K=%d must be a multiple of 8", K);
  IRON_REQUIRE(aligned16(W) && aligned16(x), "iron_gemv_bf16: W and x must be 16-byte aligned");
  IRON_REQUIRE(epilogue >= EPI_NONE && epilogue <= EPI_GELU_SIGMOID, "iron_gemv_bf16: bad epilogue %d",
               epilogue);
  GemvArgs a{static_cast<const uint16_t*>(W), nullptr, static_cast<const uint16_t*>(x),
             static_cast<uint16_t*>(y), nullptr, nullptr, nullptr, M, K, 0.f,
             epilogue};  // round-robin rows: the XCD-contiguous order measured slower for bf16 rows
  return launch_gemv_bf16<false>(a, NORM_NONE, batches, static_cast<hipStream_t>(stream));
}

static int check_norm(const char* fn, int norm_mode, const void* norm_w) {
  IRON_REQUIRE(norm_mode >= NORM_NONE && norm_mode <= NORM_SCALE, "%s: bad norm_mode %d", fn, norm_mode);
  IRON_REQUIRE((norm_mode == NORM_WEIGHT) == (norm_w != nullptr), "%s: norm_w is required for norm_mode 1 only", fn);
  return 0;
}

extern "C" int iron_gemv_bf16_fused(const void* W, const void* W2, const void* x, void* y, int M, int K,
                                    int norm_mode, const void* norm_w, float eps, const void* residual, int epilogue,
                                    void* argmax_keys, void* stream) {
  IRON_REQUIRE(W && x && y, "iron_gemv_bf16_fused: null pointer");
  IRON_REQUIRE(M > 0 && K > 0 && K % 8 == 0, "iron_gemv_bf16_fused: M=%d K=%d (K must be a multiple of 8)",
               M, K);
  IRON_REQUIRE(aligned16(W) && aligned16(x) && (!W2 || aligned16(W2)) && (!norm_w || aligned16(norm_w)),
               "iron_gemv_bf16_fused: operands must be 16-byte aligned");
  if (int rc = check_norm("iron_gemv_bf16_fused", norm_mode, norm_w)) return rc;
  IRON_REQUIRE(epilogue >= EPI_NONE && epilogue <= EPI_GELU_SIGMOID, "iron_gemv_bf16_fused: bad epilogue %d",
               epilogue);
  IRON_REQUIRE(!(W2 && epilogue != EPI_NONE), "iron_gemv_bf16_fused: the SwiGLU pair takes no epilogue");
  IRON_REQUIRE(y != x, "iron_gemv_bf16_fused: y must not alias x");
  IRON_REQUIRE((reinterpret_cast<uintptr_t>(argmax_keys) & 7u) == 0, "iron_gemv_bf16_fused: keys must be 8-byte aligned");
  GemvArgs a{static_cast<const uint16_t*>(W),
             static_cast<const uint16_t*>(W2),
             static_cast<const uint16_t*>(x),
             static_cast<uint16_t*>(y),
             static_cast<const uint16_t*>(norm_w),
             static_cast<const uint16_t*>(residual),
             static_cast<unsigned long long*>(argmax_keys),
             M,
             K,
             eps,
             epilogue};  // round-robin rows (see iron_gemv_bf16)
  hipStream_t s = static_cast<hipStream_t>(stream);
  return W2 ? launch_gemv_bf16<true>(a, norm_mode, 1, s) : launch_gemv_bf16<false>(a, norm_mode, 1, s);
}

extern "C" int iron_gemv_i4g32(const void* codes, const void* scales, const void* x, void* y, int M, int K,
                               int is_signed, void* stream) {
  return iron_gemv_i4g32_fused(codes, scales, nullptr, nullptr, x, y, M, K, is_signed, NORM_NONE, nullptr, 0.f,
                               nullptr, 0, nullptr, stream);
}

extern "C" int iron_gemv_i4g32_fused(const void* codes, const void* scales, const void* codes2,
                                     const void* scales2, const void* x, void* y, int M, int K, int is_signed,
                                     int norm_mode, const void* norm_w, float eps, const void* residual, int epilogue,
                                     void* argmax_keys, void* stream) {
  IRON_REQUIRE(codes && scales && x && y, "iron_gemv_i4g32: null pointer");
  IRON_REQUIRE((codes2 == nullptr) == (scales2 == nullptr), "iron_gemv_i4g32: codes2/scales2 come together");
  IRON_REQUIRE(M > 0 && K > 0 && K % 32 == 0, "iron_gemv_i4g32: M=%d K=%d (K must be a multiple of 32)", M,
               K);
  IRON_REQUIRE(aligned16(codes) && aligned16(x) && (!codes2 || aligned16(codes2)) &&
                   (!norm_w || aligned16(norm_w)),
               "iron_gemv_i4g32: codes, x and norm weight must be 16-byte aligned");
  IRON_REQUIRE((reinterpret_cast<uintptr_t>(scales) & 1u) == 0, "iron_gemv_i4g32: scales must be 2-byte aligned");
  if (int rc = check_norm("iron_gemv_i4g32", norm_mode, norm_w)) return rc;
  IRON_REQUIRE(epilogue >= EPI_NONE && epilogue <= EPI_GELU_SIGMOID, "iron_gemv_i4g32: bad epilogue %d",
               epilogue);
  IRON_REQUIRE(!(codes2 && epilogue != EPI_NONE), "iron_gemv_i4g32: the SwiGLU pair takes no epilogue");
  IRON_REQUIRE(y != x, "iron_gemv_i4g32: y must not alias x");
  IRON_REQUIRE((reinterpret_cast<uintptr_t>(argmax_keys) & 7u) == 0, "iron_gemv_i4g32: keys must be 8-byte aligned");
  I4Args a{static_cast<const uint8_t*>(codes),
           static_cast<const uint16_t*>(scales),
           static_cast<const uint8_t*>(codes2),
           static_cast<const uint16_t*>(scales2),
           static_cast<const uint16_t*>(x),
           static_cast<uint16_t*>(y),
           static_cast<const uint16_t*>(norm_w),
           static_cast<const uint16_t*>(residual),
           static_cast<unsigned long long*>(argmax_keys),
           M,
           K,
           eps,
           epilogue,
           is_signed ? 0x43084308u : 0x43004300u,
           is_signed ? 136.f : 128.f};
  hipStream_t s = static_cast<hipStream_t>(stream);
  return codes2 ? launch_gemv_i4<true>(a, norm_mode, s) : launch_gemv_i4<false>(a, norm_mode, s);
}

extern "C" int iron_llama_decode_head(const void* W, const void* codes, const void* scales, const void* x,
                                      void* logits, int M, int K, float eps, void* argmax_keys, unsigned* epoch,
                                      void* stream) {
  IRON_REQUIRE((W != nullptr) != (codes != nullptr), "iron_llama_decode_head: give W (bf16) or codes (int4), not both");
  IRON_REQUIRE(x && logits && argmax_keys && epoch, "iron_llama_decode_head: null pointer");
  IRON_REQUIRE(M > 0 && K > 0 && K % 32 == 0, "iron_llama_decode_head: M=%d K=%d (K must be a multiple of 32)", M, K);
  IRON_REQUIRE(aligned16(x) && (!W || aligned16(W)) && (!codes || (aligned16(codes) && scales)),
               "iron_llama_decode_head: operands must be 16-byte aligned (int4 needs its scales)");
  IRON_REQUIRE(logits != x, "iron_llama_decode_head: logits must not alias x");
  IRON_REQUIRE((reinterpret_cast<uintptr_t>(argmax_keys) & 7u) == 0 && (reinterpret_cast<uintptr_t>(epoch) & 3u) == 0,
               "iron_llama_decode_head: keys must be 8-byte and epoch 4-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (W) {
    GemvArgs a{static_cast<const uint16_t*>(W), nullptr, static_cast<const uint16_t*>(x), static_cast<uint16_t*>(logits),
               nullptr, nullptr, static_cast<unsigned long long*>(argmax_keys), M, K, eps, EPI_NONE, epoch};
    return launch_gemv_bf16<false>(a, NORM_SCALE, 1, s);
  }
  I4Args a{static_cast<const uint8_t*>(codes), static_cast<const uint16_t*>(scales), nullptr, nullptr,
           static_cast<const uint16_t*>(x), static_cast<uint16_t*>(logits), nullptr, nullptr,
           static_cast<unsigned long long*>(argmax_keys), M, K, eps, EPI_NONE, 0x43084308u, 136.f, epoch};
  return launch_gemv_i4<false>(a, NORM_SCALE, s);
}

extern "C" int iron_dequant_i4(const void* codes, const void* scales, void* out, int N, int K, int group,
                               int is_signed, void* stream) {
  IRON_REQUIRE(codes && scales && out, "iron_dequant_i4: null pointer");
  IRON_REQUIRE(N > 0 && K > 0 && K % 8 == 0, "iron_dequant_i4: N=%d K=%d (K must be a multiple of 8)", N, K);
  IRON_REQUIRE(group > 0 && group % 2 == 0 && K % group == 0,
               "iron_dequant_i4: group=%d must be even and divide K=%d", group, K);
  IRON_REQUIRE(aligned16(out) && (reinterpret_cast<uintptr_t>(codes) & 3u) == 0,
               "iron_dequant_i4: out must be 16-byte and codes 4-byte aligned");
  const size_t threads = static_cast<size_t>(N) * (K / 8);
  IRON_LAUNCH(dequant_planar_kernel, dim3((threads + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(codes),
                     static_cast<const uint16_t*>(scales), static_cast<uint16_t*>(out), N, K, group, is_signed);
  return check_launch("dequant_i4");
}

extern "C" int iron_dequant_i4_payload(const void* payload, void* out, long long size, int tile_size,
                                       int group_size, int is_signed, void* stream) {
  IRON_REQUIRE(payload && out, "iron_dequant_i4_payload: null pointer");
  IRON_REQUIRE(size > 0 && tile_size > 0 && group_size > 0, "iron_dequant_i4_payload: sizes must be positive");
  IRON_REQUIRE(size % tile_size == 0, "iron_dequant_i4_payload: size %lld must be a multiple of tile_size %d",
               size, tile_size);
  IRON_REQUIRE(tile_size % group_size == 0 && group_size % 2 == 0,
               "iron_dequant_i4_payload: group_size %d must be even and divide tile_size %d", group_size,
               tile_size);
  const long long threads = size / 2;
  IRON_LAUNCH(dequant_payload_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(payload),
                     static_cast<uint16_t*>(out), size, tile_size, group_size, is_signed);
  return check_launch("dequant_i4_payload");
}

// ---------------------------------------------------------------------------
// Symmetric int4 group-32 quantiser (weight preparation, not on the hot
// path): per group of 32, scale = bf16(max|w| / 7), q = clamp(rint(w / scale),
// -8, 7), packed two per byte along K, low nibble first.
// ---------------------------------------------------------------------------
namespace iron {
namespace {
__global__ __launch_bounds__(256) void quantize_i4g32_kernel(const uint16_t* __restrict__ W, uint8_t* __restrict__ codes,
                                                             uint16_t* __restrict__ scales, long long groups) {
  const long long g = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (g >= groups) return;
  const uint4* src = reinterpret_cast<const uint4*>(W + g * 32);
  float v[32];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 c = src[q];
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[q * 8 + 2 * e] = lo_bf16(w[e]);
      v[q * 8 + 2 * e + 1] = hi_bf16(w[e]);
    }
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, 1e-8f);
  const uint16_t sb = f32_to_bf16(amax / 7.0f);
  const float s = bf16_to_f32(sb);
  uint32_t packed[4] = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    float q = rintf(v[i] / s);
    q = fminf(fmaxf(q, -8.f), 7.f);
    const uint32_t nib = static_cast<uint32_t>(static_cast<int>(q)) & 0xfu;
    packed[i >> 3] |= nib << (4 * (i & 7));
  }
  reinterpret_cast<uint4*>(codes + g * 16)[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  scales[g] = sb;
}
}  // namespace
}  // namespace iron

extern "C" int iron_quantize_i4g32(const void* W, void* codes, void* scales, int N, int K, void* stream) {
  IRON_REQUIRE(W && codes && scales, "iron_quantize_i4g32: null pointer");
  IRON_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "iron_quantize_i4g32: N=%d K=%d (K must be a multiple of 32)", N, K);
  IRON_REQUIRE(aligned16(W) && aligned16(codes), "iron_quantize_i4g32: W and codes must be 16-byte aligned");
  const long long groups = static_cast<long long>(N) * (K / 32);
  IRON_LAUNCH(quantize_i4g32_kernel, dim3(static_cast<unsigned>((groups + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(W), static_cast<uint8_t*>(codes),
                     static_cast<uint16_t*>(scales), groups);
  return check_launch("quantize_i4g32");
}
