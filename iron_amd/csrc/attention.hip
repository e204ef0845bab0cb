// GQA attention for decode (split-K flash-decode in one kernel) and causal prefill.
//
// Decode: one new token. A workgroup owns (KV head j, a chunk of 64 cache
// positions) and serves the G = H/Hkv query heads that share KV head j, so
// every K/V byte is read from HBM once for all of them. Inside the chunk the
// softmax is exact in fp32 (scores scaled by log2(e)/sqrt(D), exp2); the
// chunk's unnormalised output, maximum and sum go to a workspace, and a second
// small kernel merges the chunks. (Merging in the last-arriving workgroup was
// measured slower: cross-XCD visibility of the partials needs either an
// agent-scope release, which writes back the whole per-XCD L2 and serialises
// across workgroups, or write-through stores plus an arrival atomic per
// workgroup, whose round trips and same-address serialisation cost more than
// the second launch.)
// RoPE for q and the new k is applied on load (two-halves rotation, row `pos`
// of an fp32 [cos, sin] interleaved table, result rounded to bf16 as the RoPE
// operator does), and the new k/v are written into the caches at `pos` by the
// workgroup whose chunk holds `pos`.
//
// Cache layout: (Hkv, max_len, D) bf16, position-major within a head, so a
// chunk of one head is one contiguous 8 KiB block.
#include "iron_common.hpp"
#include "../../include/iron_hip.h"

#include <mutex>
#include <type_traits>

namespace iron {
namespace {

constexpr int kDecChunk = 64;  // cache positions per workgroup (4 waves x 16)
constexpr int kDecThreads = 256;
constexpr int kD = 64;         // head dim (the reference MHA supports d = 64 only)

struct DecodeArgs {
  const uint16_t* q;      // (H, D) un-rotated
  const uint16_t* k_new;  // (Hkv, D) un-rotated
  const uint16_t* v_new;  // (Hkv, D)
  uint16_t* k_cache;      // (Hkv, max_len, D)
  uint16_t* v_cache;      // (Hkv, max_len, D)
  const float* angles;    // (angle_rows, D) [cos0, sin0, cos1, sin1, ...]
  uint16_t* out;          // (H, D)
  float* part;            // (Hkv, nsplit, G*D + 2G) partials
  const int* pos_dev;     // optional device-resident position (overrides pos)
  int pos;
  int max_len;
  int angle_rows;
  int nsplit;             // gridDim.x
  float scale_log2;       // log2(e) * scale
};

template <int G>
constexpr int part_stride() {
  return G * kD + 2 * G;
}

// Loads of one 16-byte chunk as 8 floats.
__device__ __forceinline__ void unpack8(const uint4 v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = lo_bf16(w[e]);
    f[2 * e + 1] = hi_bf16(w[e]);
  }
}

// Two-halves RoPE of the 8 dims of chunk c of a 64-vector, given that chunk
// (own) and chunk c ^ 4 (pair), and the 16 table floats [cos, sin] x 8 of dims
// (c & 3) * 8 + e. Lower half: x1 c - x2 s; upper half: x2 c + x1 s. Rounded
// to bf16, as the RoPE operator stores it.
__device__ __forceinline__ void rope_chunk(const uint4 own, const uint4 pair, const float* ang, bool lower, float* out) {
  float xo[8], xp[8];
  unpack8(own, xo);
  unpack8(pair, xp);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = ang[2 * e], s = ang[2 * e + 1];
    const float r = lower ? xo[e] * c - xp[e] * s : xo[e] * c + xp[e] * s;
    out[e] = bf16_to_f32(f32_to_bf16(r));
  }
}

// Lanes l and l ^ 32 of a and b summed in one exchange (v_permlane32_swap_b32
// swaps the upper 32 lanes of its first operand with the lower 32 of its
// second): lanes 0..31 return a[l] + a[l ^ 32], lanes 32..63 b[l] + b[l ^ 32].
// Inline assembly: this compiler's builtins for the permlane swaps return the
// first result in place of the second (seen in the generated code). The s_nop
// covers the VALU-write to permlane-read hazard.
__device__ __forceinline__ float fold32(float a, float b) {
  unsigned x = __builtin_bit_cast(unsigned, a), y = __builtin_bit_cast(unsigned, b);
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  return __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
}

// The same over lanes l and l ^ 16 (v_permlane16_swap_b32 swaps the odd
// 16-lane rows of its first operand with the even rows of its second): rows 0
// and 2 return a[l] + a[l ^ 16], rows 1 and 3 b[l] + b[l ^ 16].
__device__ __forceinline__ float fold16(float a, float b) {
  unsigned x = __builtin_bit_cast(unsigned, a), y = __builtin_bit_cast(unsigned, b);
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  return __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
}

// 2^x by v_exp_f32 alone, for x <= 0 (softmax weights): results below 2^-126
// flush to zero, which the weights tolerate; elsewhere exp2f's value.
__device__ __forceinline__ float exp2_weight(float x) { return __builtin_amdgcn_exp2f(x); }

// One decode step of KV head j (blockIdx.y) for its G query heads; workgroup
// s (blockIdx.x) owns cache positions [64 s, 64 s + 64).
//
// Wave w of the workgroup takes positions 64 s + 16 w + [0, 16): lane
// (r = lane / 8, c = lane % 8) holds rows r and r + 8 of them, dims 8c..8c+7.
// Every global load (K/V rows, q and the table row, the owner's new k/v) is
// issued as soon as `pos` is known. q is rotated once per workgroup (one
// element per thread) into LDS as bf16. Scores are bf16 dot products
// (v_dot2_f32_bf16: exact products, fp32 sums) summed over the 8 lanes of a
// row by DPP; the softmax statistics of the wave's 16 rows come from wave-wide
// DPP reductions, and the wave's unnormalised output (G x 64 values, 8G per
// lane) is summed over the 8 rows of lanes with two permlane folds and one
// DPP step, which leave each lane 2G totals. The four waves meet once in LDS
// to form the chunk's partial (output, maximum, sum), written to the
// workspace for gqa_combine_kernel.
template <int G>
__global__ __launch_bounds__(kDecThreads) void gqa_decode_kernel(DecodeArgs a) {
  constexpr int D = kD;
  constexpr int NW = kDecThreads / kWave;
  constexpr int PS = part_stride<G>();
  constexpr int NV = 8 * G;  // unnormalised output values per lane before the folds
  __shared__ __attribute__((aligned(16))) uint16_t q_s[G * D];  // rotated q, bf16
  __shared__ float wm_s[NW][G], wl_s[NW][G];
  __shared__ __attribute__((aligned(16))) float wo_s[NW][G * D];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid >> 6;
  const int s = blockIdx.x, j = blockIdx.y;
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  if (pos < 0 || pos >= a.max_len || pos >= a.angle_rows) return;  // rejected on the host when pos is known
  const int L = pos + 1;
  const int p0 = s * kDecChunk;
  if (p0 >= L) return;
  const int c = lane & 7, r = lane >> 3;
  const bool lower = c < 4;
  const int wrow0 = p0 + 16 * w;
  const bool owner = pos >= wrow0 && pos < wrow0 + 16;

  // cache rows: unconditional loads of a clamped row (a guarded load compiled
  // to a branch that waited for its data); rows >= pos are replaced below
  // (the new token) or masked (past it)
  uint4 kraw[2], vraw[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = min(wrow0 + r + 8 * h, a.max_len - 1);
    const size_t off = (static_cast<size_t>(j) * a.max_len + p) * D + c * 8;
    kraw[h] = ld_stream16(a.k_cache + off);
    vraw[h] = ld_stream16(a.v_cache + off);
  }
  const float* angrow = a.angles + static_cast<size_t>(pos) * D;
  float ang[16];
  uint4 kna = make_uint4(0, 0, 0, 0), knb = kna, vn = kna;
  if (owner) {  // the new token's table entries and k/v, in flight with the cache rows
    const float4* ap = reinterpret_cast<const float4*>(angrow + (c & 3) * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 t = ap[i];
      ang[4 * i] = t.x;
      ang[4 * i + 1] = t.y;
      ang[4 * i + 2] = t.z;
      ang[4 * i + 3] = t.w;
    }
    kna = *reinterpret_cast<const uint4*>(a.k_new + static_cast<size_t>(j) * D + c * 8);
    knb = *reinterpret_cast<const uint4*>(a.k_new + static_cast<size_t>(j) * D + (c ^ 4) * 8);
    vn = *reinterpret_cast<const uint4*>(a.v_new + static_cast<size_t>(j) * D + c * 8);
  }
  const uint16_t* qh = a.q + static_cast<size_t>(j) * G * D;
  for (int t = tid; t < G * D; t += kDecThreads) {
    const int d = t % D, i = d & 31;
    const float x = bf16_to_f32(qh[t]), xp = bf16_to_f32(qh[t ^ 32]);
    const float cs = angrow[2 * i], sn = angrow[2 * i + 1];
    q_s[t] = f32_to_bf16(d < 32 ? x * cs - xp * sn : x * cs + xp * sn);
  }
  __syncthreads();
  uint4 qk[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qk[g] = *reinterpret_cast<const uint4*>(&q_s[g * D + c * 8]);

  // One code path for waves whose 16 rows are all valid and none is the new
  // token (every wave but the last one or two), one with the masks and the
  // owner's append.
  const bool full = wrow0 + 16 <= L && !owner;  // wave-uniform
  auto wave_body = [&](auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    // K rows as packed bf16, V rows as floats (zero past pos: 0 * stale data must not reach o)
    uint32_t kw[2][4];
    float vf[2][8];
    bool valid[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int p = wrow0 + r + 8 * h;
      valid[h] = FULL || p < L;
      if (!FULL && p == pos) {  // the new token: rotate k, append k/v to the caches
        float kr[8];
        rope_chunk(kna, knb, ang, lower, kr);
#pragma unroll
        for (int e = 0; e < 4; ++e) kw[h][e] = pack_bf16x2(kr[2 * e], kr[2 * e + 1]);  // exact: bf16 values
        unpack8(vn, vf[h]);
        const size_t off = (static_cast<size_t>(j) * a.max_len + pos) * D + c * 8;
        *reinterpret_cast<uint4*>(a.k_cache + off) = make_uint4(kw[h][0], kw[h][1], kw[h][2], kw[h][3]);
        *reinterpret_cast<uint4*>(a.v_cache + off) = vn;
      } else {
        kw[h][0] = kraw[h].x;
        kw[h][1] = kraw[h].y;
        kw[h][2] = kraw[h].z;
        kw[h][3] = kraw[h].w;
        unpack8(vraw[h], vf[h]);
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[h][e] = FULL || valid[h] ? vf[h][e] : 0.f;
      }
    }

    // scores in the log2 domain; the 8 lanes of a row sum their partial dots
    float sc[2][G];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = dot2_bf16(qk[g].x, kw[h][0], 0.f);
        d = dot2_bf16(qk[g].y, kw[h][1], d);
        d = dot2_bf16(qk[g].z, kw[h][2], d);
        d = dot2_bf16(qk[g].w, kw[h][3], d);
        d = add_dpp<0xB1>(d);   // + lane ^ 1
        d = add_dpp<0x4E>(d);   // + lane ^ 2
        d = add_dpp<0x141>(d);  // + lane 7-i of the 8: full 8-lane sum
        sc[h][g] = FULL || valid[h] ? d * a.scale_log2 : -INFINITY;
      }

    // the wave's statistics and unnormalised output over its 16 rows
    float ov[NV];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m = wave_max(fmaxf(sc[0][g], sc[1][g]));  // -inf only when all 16 rows are past pos
      const float e0 = FULL || valid[0] ? exp2_weight(sc[0][g] - m) : 0.f;
      const float e1 = FULL || valid[1] ? exp2_weight(sc[1][g] - m) : 0.f;
      const float l = wave_sum(c == 0 ? e0 + e1 : 0.f);
      if (lane == 0) {
        wm_s[w][g] = m;
        wl_s[w][g] = l;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ov[g * 8 + e] = fmaf(e0, vf[0][e], e1 * vf[1][e]);
    }
    // sum over the 8 rows r (lane bits 3..5): value k pairs with k + NV/2 across
    // lane bit 5, then with k + NV/4 across bit 4, then a DPP step over bit 3
    float o2[NV / 2], o4[NV / 4];
#pragma unroll
    for (int k = 0; k < NV / 2; ++k) o2[k] = fold32(ov[k], ov[k + NV / 2]);
#pragma unroll
    for (int k = 0; k < NV / 4; ++k) {
      const float t = fold16(o2[k], o2[k + NV / 4]);
      o4[k] = t + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x128, 0xf,
                                                                            0xf, false));  // row_ror:8 = lane ^ 8
    }
    // lane holds totals k = (lane bit 5) NV/2 + (lane bit 4) NV/4 + [0, NV/4): value k is (g = k / 8, dim 8c + k % 8)
    if (((lane >> 3) & 1) == 0) {
      const int k0 = (lane >> 5) * (NV / 2) + ((lane >> 4) & 1) * (NV / 4);
#pragma unroll
      for (int k = 0; k < NV / 4; ++k) {
        const int kk = k0 + k;
        wo_s[w][(kk / 8) * D + c * 8 + kk % 8] = o4[k];
      }
    }
  };
  if (full)
    wave_body(std::true_type{});
  else
    wave_body(std::false_type{});
  __syncthreads();

  // the chunk's partial: the four waves merged
  float* part = a.part + (static_cast<size_t>(j) * a.nsplit + s) * PS;
  for (int t = tid; t < G * D; t += kDecThreads) {
    const int g = t / D;
    float M = wm_s[0][g];  // finite: position p0 < L is in wave 0
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) M = fmaxf(M, wm_s[ww][g]);
    float o = 0.f, l = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float f = exp2_weight(wm_s[ww][g] - M);  // 0 for a wave whose rows are all past pos
      o = fmaf(f, wo_s[ww][t], o);
      l = fmaf(f, wl_s[ww][g], l);
    }
    part[t] = o;
    if (t % D == 0) {
      part[G * D + g] = M;
      part[G * D + G + g] = l;
    }
  }
}

// Merge of the chunk partials, one 1024-thread workgroup per query head
// (Hkv * G workgroups). Thread -> output dim d of the head and slice q of the
// chunks (chunks q, q + 16, ...). Each thread folds its chunks with a running
// maximum, loading 8 chunks per step with every load in flight (one step
// covers 128 chunks, i.e. 8192 positions); the 16 slices are then combined
// through LDS.
constexpr int kMergeThreads = 1024;

template <int G>
__global__ __launch_bounds__(kMergeThreads) void gqa_combine_kernel(DecodeArgs a) {
  constexpr int D = kD;
  constexpr int PS = part_stride<G>();
  constexpr int NQ = kMergeThreads / D;  // chunk slices
  constexpr int B = 8;                   // chunks per step per thread
  __shared__ float m_s[kMergeThreads], l_s[kMergeThreads], o_s[kMergeThreads];
  const int tid = threadIdx.x, d = tid % D, q = tid / D;
  const int h = blockIdx.x, j = h / G, g = h % G;
  const float* base = a.part + static_cast<size_t>(j) * a.nsplit * PS;
  // The first B chunks of this slice are loaded before the position is known
  // (any chunk < nsplit is inside the workspace); chunks past the active count
  // are dropped by selects below, so stale workspace values never mix in.
  // (Unconditional loads of a clamped chunk index: a guarded load compiled to
  // a branch that waited for its data before the next chunk's loads.)
  float mb[B], lb[B], ob[B];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const float* pk = base + static_cast<size_t>(min(q + b * NQ, a.nsplit - 1)) * PS;
    mb[b] = pk[G * D + g];
    lb[b] = pk[G * D + G + g];
    ob[b] = pk[g * D + d];
  }
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  if (pos < 0 || pos >= a.max_len || pos >= a.angle_rows) return;
  const int nact = (pos + kDecChunk) / kDecChunk;
  float M = -INFINITY, Ls = 0.f, acc = 0.f;
  for (int k0 = q; k0 < nact; k0 += NQ * B) {
    if (k0 != q) {
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const float* pk = base + static_cast<size_t>(min(k0 + b * NQ, nact - 1)) * PS;
        mb[b] = pk[G * D + g];
        lb[b] = pk[G * D + G + g];
        ob[b] = pk[g * D + d];
      }
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {  // chunks past the active count (or stale ones) weigh nothing
      const bool live = k0 + b * NQ < nact;
      mb[b] = live ? mb[b] : -INFINITY;
      lb[b] = live ? lb[b] : 0.f;
      ob[b] = live ? ob[b] : 0.f;
    }
    float bm = M;
#pragma unroll
    for (int b = 0; b < B; ++b) bm = fmaxf(bm, mb[b]);  // finite: chunk k0 < nact is active
    const float keep = exp2f(M - bm);                   // 0 on the first step
    acc *= keep;
    Ls *= keep;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float w = exp2f(mb[b] - bm);  // 0 for the chunks past nact
      acc = fmaf(w, ob[b], acc);
      Ls = fmaf(w, lb[b], Ls);
    }
    M = bm;
  }
  m_s[tid] = M;
  l_s[tid] = Ls;
  o_s[tid] = acc;
  __syncthreads();
  if (q == 0) {
    float Mx = M;  // slice 0 always holds chunk 0
#pragma unroll
    for (int qq = 1; qq < NQ; ++qq) Mx = fmaxf(Mx, m_s[qq * D + d]);
    float lt = 0.f, ot = 0.f;
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
      const float w = exp2f(m_s[qq * D + d] - Mx);  // 0 for an empty slice
      lt = fmaf(w, l_s[qq * D + d], lt);
      ot = fmaf(w, o_s[qq * D + d], ot);
    }
    a.out[static_cast<size_t>(h) * D + d] = f32_to_bf16(ot / lt);
  }
}

// Merge of the chunk partials with one wave per query head (Hkv * G
// workgroups of 64 threads): lane i holds the statistics (maximum, sum) of
// chunks i, i + 64, ..., lane d accumulates output dim d, and each chunk's
// weight reaches every lane by readlane. The loads of the first 64 chunks are
// issued before the position is read, so a context of up to 4096 positions
// costs one memory round trip. Chunks past the active count are dropped by
// selects (their workspace may hold anything).
template <int G>
__global__ __launch_bounds__(kWave) void gqa_merge_kernel(DecodeArgs a) {
  constexpr int D = kD;
  constexpr int PS = part_stride<G>();
  const int lane = threadIdx.x;
  const int h = blockIdx.x, j = h / G, g = h % G;
  const float* base = a.part + static_cast<size_t>(j) * a.nsplit * PS;
  const float* pl = base + static_cast<size_t>(min(lane, a.nsplit - 1)) * PS;
  float mb = pl[G * D + g], lb = pl[G * D + G + g];
  float ob[kWave];
#pragma unroll
  for (int u = 0; u < kWave; ++u) ob[u] = base[static_cast<size_t>(min(u, a.nsplit - 1)) * PS + g * D + lane];
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  if (pos < 0 || pos >= a.max_len || pos >= a.angle_rows) return;
  const int nact = (pos + kDecChunk) / kDecChunk;
  float M = lane < nact ? mb : -INFINITY;
  for (int i = lane + kWave; i < nact; i += kWave) M = fmaxf(M, base[static_cast<size_t>(i) * PS + G * D + g]);
  M = wave_max(M);  // finite: chunk 0 is active
  float acc = 0.f, Ls = 0.f;
  for (int b0 = 0; b0 < nact; b0 += kWave) {
    if (b0 > 0) {  // contexts past 64 chunks: the next 64
      const float* pb = base + static_cast<size_t>(min(b0 + lane, nact - 1)) * PS;
      mb = pb[G * D + g];
      lb = pb[G * D + G + g];
#pragma unroll
      for (int u = 0; u < kWave; ++u) ob[u] = base[static_cast<size_t>(min(b0 + u, nact - 1)) * PS + g * D + lane];
    }
    const bool live = b0 + lane < nact;
    const float wgt = live ? exp2f(mb - M) : 0.f;
    Ls = fmaf(wgt, live ? lb : 0.f, Ls);
#pragma unroll
    for (int u = 0; u < kWave; ++u) {
      const float wu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), u));
      acc = fmaf(wu, b0 + u < nact ? ob[u] : 0.f, acc);
    }
  }
  Ls = wave_sum(Ls);
  a.out[static_cast<size_t>(h) * D + lane] = f32_to_bf16(acc / Ls);
}

// ---------------------------------------------------------------------------
// Prefill / MHA: causal (optional) flash attention over strided Q, K, V on
// MFMA (v_mfma_f32_32x32x16_bf16).
//
// Workgroup = 4 waves = 128 queries of one head; each wave owns 32 queries and
// walks the visible keys in blocks of 64. K and V blocks are staged row-major
// in a 3-stage LDS ring filled by global_load_lds_dwordx4 (no VGPR staging, no
// LDS stores), two blocks ahead of the one being computed, one barrier per
// block. Per block a wave computes S^T = K Q^T (two 32x32 tiles): every lane
// then holds one query column (lane % 32) and 16 keys, so the softmax row
// statistics need only the lane's own registers and one exchange with lane ^ 32.
// The probabilities go to bf16 and feed O^T += V^T P^T directly from registers
// as the B operand; the k index of that product is a permutation of the
// block's keys that matches the S^T accumulator layout. The V^T operand comes
// straight from the row-major V block through ds_read_b64_tr_b16: in each
// 16-lane group, lane i receives element i % 4 of the 8-byte rows addressed by
// lanes 4j + i / 4 (j = 0..3), so lanes addressing 4 keys x 16 dims receive 16
// dims x 4 keys. K rows keep the 16-byte chunk c at slot c ^ ((key / 2) % 8)
// (16 rows of a ds_read_b128 on distinct banks); V rows at slot
// c ^ (((key / 2) % 2) * 4): a transposed read serves 32 lanes per LDS pass,
// 4 rows x 4 chunks, and this maps rows r and r + 2 to disjoint slot halves
// (with rows r and r + 1 on opposite bank halves, all 64 banks once).
// Online softmax in the log2 domain, fp32 statistics; output rows in
// [Sq, out_rows) are zero-filled (the MHA operator's padding).
// ---------------------------------------------------------------------------
struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  long long q_hs, q_rs;  // element strides: per head, per row
  long long k_hs, k_rs;
  long long v_hs, v_rs;
  long long o_hs, o_rs;
  int H, Hkv, Sq, Skv;
  int out_rows;  // rows of out to write; rows in [Sq, out_rows) are zero-filled
  int causal;
  int q_offset;  // absolute position of query row 0 (keys <= it are visible)
  float scale_log2;
};

typedef __bf16 fa_bf16x8 __attribute__((ext_vector_type(8)));
typedef float fa_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int fa_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int fa_u32x2 __attribute__((ext_vector_type(2)));

typedef short fa_i16x4 __attribute__((ext_vector_type(4)));

constexpr int kFaQ = 128;             // queries per workgroup (4 waves x 32)
constexpr int kFaK = 64;              // keys per block
constexpr int kFaStages = 4;          // K/V blocks resident (see the pipeline in the kernel)
constexpr int kFaBlock = kFaK * 128;  // bytes of a 64-row K (or V) block
constexpr int kOutStride = 72;        // output staging row (144 B)
constexpr int kFaLds = (kFaStages * 2 * kFaBlock) > (4 * 32 * kOutStride * 2) ? (kFaStages * 2 * kFaBlock)
                                                                               : (4 * 32 * kOutStride * 2);

// Lanes l and l ^ 32 exchange values in one VALU op (v_permlane32_swap_b32
// swaps the upper half of its first operand with the lower half of its
// second): with both operands x, the two results hold x[l] and x[l ^ 32] in
// every lane. Inline assembly, because the compiler's builtin for it kept only
// the first of the two results here. The s_nop covers the VALU-write to
// permlane-read hazard (the compiler emits the same before the builtin).
__device__ __forceinline__ void fa_pair(float x, float& r0, float& r1) {
  unsigned a = __builtin_bit_cast(unsigned, x), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  r0 = __builtin_bit_cast(float, a);
  r1 = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float fa_pair_max(float x) {
  float r0, r1;
  fa_pair(x, r0, r1);
  return fmaxf(r0, r1);
}
__device__ __forceinline__ float fa_pair_sum(float x) {
  float r0, r1;
  fa_pair(x, r0, r1);
  return r0 + r1;
}

__device__ __forceinline__ int fa_k_slot(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }
__device__ __forceinline__ int fa_v_slot(int row, int chunk) { return chunk ^ (((row >> 1) & 1) << 2); }

// Wait until at most N of this wave's global loads are outstanding, then
// barrier (__syncthreads would wait for all of them). The memory clobber keeps
// the next stage's LDS reads below the barrier.
template <int N>
__device__ __forceinline__ void fa_wait_loads_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

__global__ __launch_bounds__(256) void attention_prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kFaLds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hh = lane >> 5;
  // Workgroup order: x = head, y = query tile. Causal tiles run heaviest
  // first (the last tile sees the most keys), and when H % 8 == 0 the heads
  // are permuted so that each XCD (workgroup b runs on XCD b % 8) holds
  // H / 8 consecutive heads, which share KV heads and so K/V blocks in its L2.
  const int bx = blockIdx.x;
  const int h = (a.H % 8 == 0) ? (bx % 8) * (a.H / 8) + bx / 8 : bx;
  const int hk = h / (a.H / a.Hkv);
  const int tile = a.causal ? static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y) : blockIdx.y;
  const int q0 = tile * kFaQ;
  if (q0 >= a.Sq) {  // padding rows only (uniform per workgroup)
    for (int e = tid; e < kFaQ * (kD / 8); e += 256) {
      const int r = q0 + (e >> 3), ch = e & 7;
      if (r < a.out_rows)
        *reinterpret_cast<fa_u32x4*>(a.out + h * a.o_hs + static_cast<long long>(r) * a.o_rs + ch * 8) =
            fa_u32x4{0, 0, 0, 0};
    }
    return;
  }
  const int qw = q0 + wave * 32;  // this wave's first query row

  // Q fragments (B operand of S^T): query qw + c, dims 16 kk + 8 hh .. + 8
  fa_bf16x8 qf[4];
  {
    const int qrow = min(qw + c, a.Sq - 1);
    const uint16_t* qp = a.q + h * a.q_hs + static_cast<long long>(qrow) * a.q_rs;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      qf[kk] = __builtin_bit_cast(fa_bf16x8, *reinterpret_cast<const fa_u32x4*>(qp + 16 * kk + 8 * hh));
  }
  fa_f32x16 o[2];
#pragma unroll
  for (int j = 0; j < 16; ++j) o[0][j] = o[1][j] = 0.f;
  float m = -INFINITY, l = 0.f;
  const int qpos = a.q_offset + qw + c;  // absolute position of this lane's query
  int kend = a.Skv;
  if (a.causal) kend = min(kend, a.q_offset + min(q0 + kFaQ, a.Sq));
  const int nb = (kend + kFaK - 1) / kFaK;
  const int wave_last = a.q_offset + min(qw + 31, a.Sq - 1);
  const int wave_first = a.q_offset + qw;  // keys <= it are visible to every query of the wave

  // Loader: a stage is [K block][V block], each 8 x 1 KiB of 8 rows; wave w
  // loads 1 KiB blocks 4w..4w+3 (0-7 K, 8-15 V). Lane l lands on row
  // 8 (b % 8) + l / 8, slot l % 8 and fetches the chunk that belongs there.
  // Keys past Skv load key Skv-1: finite values whose weights are zero.
  // Blocks are issued in order 0, 1, 2, ...: each lane keeps the source of
  // its next row and bumps it by 64 rows per issue; only a block that runs
  // past Skv recomputes clamped addresses.
  const uint16_t* src[4];
  const uint16_t* next_src[4];
  long long rstride[4];
  int lrow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = wave * 4 + j;
    const bool is_k = b < 8;
    const int r = (b & 7) * 8 + (lane >> 3), slot = lane & 7;
    const int chunk = is_k ? fa_k_slot(r, slot) : fa_v_slot(r, slot);  // both are involutions
    src[j] = (is_k ? a.k + hk * a.k_hs : a.v + hk * a.v_hs) + chunk * 8;
    rstride[j] = is_k ? a.k_rs : a.v_rs;
    lrow[j] = r;
    next_src[j] = src[j] + r * rstride[j];
  }
  auto issue = [&](int bi) {
    unsigned char* st = lds + (bi % kFaStages) * 2 * kFaBlock;
    const bool inside = bi * kFaK + kFaK <= a.Skv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t* p = inside ? next_src[j] : src[j] + min(bi * kFaK + lrow[j], a.Skv - 1) * rstride[j];
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const unsigned*>(p),
                                       reinterpret_cast<unsigned*>(st + (wave * 4 + j) * 1024), 16, 0, 0);
      next_src[j] += kFaK * rstride[j];
    }
  };
  // this lane's transposed-read address inside a V block: 16-lane group g
  // covers dims 16 (g % 2) .. + 15 (+ 32 db) and keys 4 hh .. + 3 (+ 16 st, + 8)
  const int tr_row = 4 * hh + ((lane & 15) >> 2), tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // S^T = K Q^T for block bi: sc[b][j] is key 64 bi + 32 b + 8 (j / 4) + 4 hh + j % 4, query qw + c
  auto scores = [&](int bi, fa_f32x16 (&sc)[2]) {
    const unsigned char* ks = lds + (bi % kFaStages) * 2 * kFaBlock;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int kr = 32 * b + c;
      fa_f32x16 acc = {};  // the first MFMA takes an inline zero accumulator
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const fa_bf16x8 kf = __builtin_bit_cast(
            fa_bf16x8, *reinterpret_cast<const fa_u32x4*>(ks + kr * 128 + fa_k_slot(kr, 2 * kk + hh) * 16));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], acc, 0, 0, 0);
      }
      sc[b] = acc;
    }
  };
  auto visible = [&](int bi) { return !a.causal || bi * kFaK <= wave_last; };

  // Software pipeline over key blocks: iteration bi waits for block bi+1,
  // issues its S^T MFMAs, then runs block bi's softmax and P V while they
  // execute. Stages: bi (V being read), bi+1 (K being read), bi+2 in flight,
  // bi+3 being issued into the stage block bi-1 used.
#pragma unroll
  for (int p = 0; p < kFaStages - 1; ++p)
    if (p < nb) issue(p);
  static_assert(kFaStages == 4, "the wait counts below assume 4 stages");
  if (nb >= 3)
    fa_wait_loads_barrier<8>();
  else if (nb == 2)
    fa_wait_loads_barrier<4>();
  else
    fa_wait_loads_barrier<0>();
  fa_f32x16 sa[2], sb[2];
  if (visible(0)) scores(0, sa);

  auto step = [&](int bi, fa_f32x16 (&cur)[2], fa_f32x16 (&nxt)[2]) {
    if (bi + 1 < nb) {
      if (bi + 2 < nb)
        fa_wait_loads_barrier<4>();
      else
        fa_wait_loads_barrier<0>();
      // block bi-1's stage is free: every wave passed this barrier after its last read of it
      if (bi + kFaStages - 1 < nb) issue(bi + kFaStages - 1);
      if (visible(bi + 1)) scores(bi + 1, nxt);
    }
    if (!visible(bi)) return;  // every key of the block is after this wave's queries
    const int k0 = bi * kFaK;
    const unsigned char* vs = lds + (bi % kFaStages) * 2 * kFaBlock + kFaBlock;
      // V^T fragments for O^T += V^T P^T, read while the next block's S^T MFMAs run: k-step st,
      // element i of lane (d, hh) is key 16 st + 8 (i / 4) + 4 hh + i % 4 (two
      // transposed reads of 4 keys each). The reads are inline assembly ending in
      // their own lgkmcnt wait: as a builtin, the compiler makes the first one wait
      // for every LDS-direct load in flight (it cannot tell the stages apart).
      fa_u32x2 vt[2][4][2];
      {
        const unsigned vb = static_cast<unsigned>(reinterpret_cast<uintptr_t>(vs));
        unsigned ad[2][4][2];
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const int dim = 32 * db + tr_dim;
#pragma unroll
          for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int hl = 0; hl < 2; ++hl) {
              const int r = 16 * st + 8 * hl + tr_row;
              ad[db][st][hl] = vb + r * 128 + fa_v_slot(r, dim >> 3) * 16 + (dim & 7) * 2;
            }
        }
        asm volatile(
            "ds_read_b64_tr_b16 %0, %16\n\tds_read_b64_tr_b16 %1, %17\n\t"
            "ds_read_b64_tr_b16 %2, %18\n\tds_read_b64_tr_b16 %3, %19\n\t"
            "ds_read_b64_tr_b16 %4, %20\n\tds_read_b64_tr_b16 %5, %21\n\t"
            "ds_read_b64_tr_b16 %6, %22\n\tds_read_b64_tr_b16 %7, %23\n\t"
            "ds_read_b64_tr_b16 %8, %24\n\tds_read_b64_tr_b16 %9, %25\n\t"
            "ds_read_b64_tr_b16 %10, %26\n\tds_read_b64_tr_b16 %11, %27\n\t"
            "ds_read_b64_tr_b16 %12, %28\n\tds_read_b64_tr_b16 %13, %29\n\t"
            "ds_read_b64_tr_b16 %14, %30\n\tds_read_b64_tr_b16 %15, %31\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(vt[0][0][0]), "=&v"(vt[0][0][1]), "=&v"(vt[0][1][0]), "=&v"(vt[0][1][1]), "=&v"(vt[0][2][0]),
              "=&v"(vt[0][2][1]), "=&v"(vt[0][3][0]), "=&v"(vt[0][3][1]), "=&v"(vt[1][0][0]), "=&v"(vt[1][0][1]),
              "=&v"(vt[1][1][0]), "=&v"(vt[1][1][1]), "=&v"(vt[1][2][0]), "=&v"(vt[1][2][1]), "=&v"(vt[1][3][0]),
              "=&v"(vt[1][3][1])
            : "v"(ad[0][0][0]), "v"(ad[0][0][1]), "v"(ad[0][1][0]), "v"(ad[0][1][1]), "v"(ad[0][2][0]),
              "v"(ad[0][2][1]), "v"(ad[0][3][0]), "v"(ad[0][3][1]), "v"(ad[1][0][0]), "v"(ad[1][0][1]),
              "v"(ad[1][1][0]), "v"(ad[1][1][1]), "v"(ad[1][2][0]), "v"(ad[1][2][1]), "v"(ad[1][3][0]),
              "v"(ad[1][3][1]));
      }
      // Online softmax in the log2 domain with c = scale * log2(e) > 0: the row
      // maximum is taken on the raw scores, p = 2^(s c - m) is one FMA and one
      // v_exp_f32. Only blocks that cross Skv or the causal diagonal of this
      // wave's queries are masked. The softmax VALU work, not the MFMAs,
      // bounds this loop.
      const float cs = a.scale_log2;
      float mx = -INFINITY;
      if (k0 + kFaK > a.Skv || (a.causal && k0 + kFaK - 1 > wave_first)) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = k0 + 32 * b + 8 * (j >> 2) + 4 * hh + (j & 3);
            const bool vis = key < a.Skv && (!a.causal || key <= qpos);
            cur[b][j] = vis ? cur[b][j] : -INFINITY;
            mx = fmaxf(mx, cur[b][j]);
          }
      } else {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int j = 0; j < 16; j += 2) mx = fmaxf(mx, fmaxf(cur[b][j], cur[b][j + 1]));  // v_max3_f32
      }
      mx = fa_pair_max(mx);
      // Lazy rescaling: the running maximum m moves only when this block's
      // maximum exceeds it by more than 8 (log2 units), so p = 2^(s c - m) <= 2^8
      // stays well inside bf16/fp32 range and O is rarely rescaled. The result
      // sum(p v) / sum(p) does not depend on which m is used.
      const float mblk = mx * cs;
      const bool grow = mblk > m + 8.f;  // first visible block: m = -inf
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float alpha = grow ? __builtin_amdgcn_exp2f(m - mblk) : 1.f;  // 0 when m = -inf
        m = grow ? mblk : m;
        l *= alpha;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          o[0][j] *= alpha;
          o[1][j] *= alpha;
        }
      }
      const float moff = (m == -INFINITY) ? 0.f : m;  // keeps 2^(-inf - moff) = 0, never NaN
      // P^T fragments: pf[2 b + sp] element i = register 8 sp + i of s[b]
      fa_bf16x8 pf[4];
      float psum = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int sp = 0; sp < 2; ++sp) {
          float p[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(cur[b][8 * sp + i], cs, -moff));
          const fa_u32x4 w = {cvt_pk_bf16(p[0], p[1]), cvt_pk_bf16(p[2], p[3]), cvt_pk_bf16(p[4], p[5]),
                              cvt_pk_bf16(p[6], p[7])};
          // the row sum of the bf16 weights the PV product uses, two per v_dot2
#pragma unroll
          for (int i = 0; i < 4; ++i) psum = dot2_bf16(w[i], 0x3f803f80u, psum);
          pf[2 * b + sp] = __builtin_bit_cast(fa_bf16x8, w);
        }
      l += psum;
      // O^T += V^T P^T over the block's 64 keys, 4 k-steps of 16
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const fa_u32x4 vw = {vt[db][st][0].x, vt[db][st][0].y, vt[db][st][1].x, vt[db][st][1].y};
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(fa_bf16x8, vw), pf[st], o[db], 0, 0, 0);
        }
  };
  for (int bi = 0; bi < nb; bi += 2) {
    step(bi, sa, sb);
    if (bi + 1 < nb) step(bi + 1, sb, sa);
  }

  l = fa_pair_sum(l);  // the two halves summed different keys of the same query
  const float inv = l > 0.f ? 1.f / l : 0.f;
  __syncthreads();  // every wave is done with the K/V tiles
  uint16_t* stg = reinterpret_cast<uint16_t*>(lds) + wave * 32 * kOutStride;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int d = 32 * db + 8 * (j >> 2) + 4 * hh + (j & 3);
      stg[c * kOutStride + d] = f32_to_bf16(o[db][j] * inv);
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i, r = e >> 3, ch = e & 7, q = qw + r;
    uint16_t* dst = a.out + h * a.o_hs + static_cast<long long>(q) * a.o_rs + ch * 8;
    if (q < a.Sq)
      *reinterpret_cast<fa_u32x4*>(dst) = *reinterpret_cast<const fa_u32x4*>(stg + r * kOutStride + ch * 8);
    else if (q < a.out_rows)
      *reinterpret_cast<fa_u32x4*>(dst) = fa_u32x4{0, 0, 0, 0};
  }
}

}  // namespace
}  // namespace iron

using namespace iron;

static int decode_nsplit(int max_len) { return (max_len + kDecChunk - 1) / kDecChunk; }

extern "C" long long iron_gqa_decode_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int max_len) {
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim != kD || max_len <= 0) return -1;
  const int G = n_heads / n_kv_heads;
  const long long part = static_cast<long long>(n_kv_heads) * decode_nsplit(max_len) * (G * kD + 2 * G) * 4;
  return 256 + part;  // 256 reserved bytes, then partials
}

// Checks and launches of one GQA decode step with its partials in `workspace`
// (iron_gqa_decode_workspace_bytes() of the shape, 256-byte aligned); shared
// by the entry point that takes a workspace and the one that uses the
// library's own scratch array.
static int gqa_decode_launch(const char* who, const void* q, const void* k_new, const void* v_new, void* k_cache,
                             void* v_cache, const float* angles, int angle_rows, void* out, void* workspace,
                             int n_heads, int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev,
                             float scale, void* stream) {
  IRON_REQUIRE(q && k_new && v_new && k_cache && v_cache && angles && out && workspace, "%s: null pointer", who);
  IRON_REQUIRE(head_dim == kD, "%s: head_dim=%d (only 64 is supported)", who, head_dim);
  IRON_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "%s: n_heads=%d must be a multiple of n_kv_heads=%d", who, n_heads, n_kv_heads);
  const int G = n_heads / n_kv_heads;
  IRON_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "%s: group size %d not in {1,2,4,8}", who, G);
  IRON_REQUIRE(n_kv_heads * 4 <= 256, "%s: at most 64 KV heads", who);
  IRON_REQUIRE(max_len > 0 && angle_rows > 0, "%s: max_len and angle_rows must be positive", who);
  IRON_REQUIRE(pos_dev || (pos >= 0 && pos < max_len && pos < angle_rows),
               "%s: pos=%d outside the cache (max_len=%d) or angle table (%d rows)", who, pos, max_len, angle_rows);
  IRON_REQUIRE(aligned16(q) && aligned16(k_new) && aligned16(v_new) && aligned16(k_cache) && aligned16(v_cache) &&
                   aligned16(angles),
               "%s: q, k_new, v_new, the caches and the angle table must be 16-byte aligned", who);
  IRON_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "%s: workspace must be 256-byte aligned", who);
  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.angles = angles;
  a.out = static_cast<uint16_t*>(out);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
  a.pos_dev = pos_dev;
  a.pos = pos;
  a.max_len = max_len;
  a.angle_rows = angle_rows;
  a.nsplit = decode_nsplit(max_len);
  a.scale_log2 = scale * 1.4426950408889634f;
  dim3 grid(a.nsplit, n_kv_heads), block(kDecThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 cgrid(n_kv_heads * G), cblock(kMergeThreads);
  switch (G) {
    case 1:
      IRON_LAUNCH((gqa_decode_kernel<1>), grid, block, 0, s, a);
      IRON_LAUNCH((gqa_combine_kernel<1>), cgrid, cblock, 0, s, a);
      break;
    case 2:
      IRON_LAUNCH((gqa_decode_kernel<2>), grid, block, 0, s, a);
      IRON_LAUNCH((gqa_combine_kernel<2>), cgrid, cblock, 0, s, a);
      break;
    case 4:
      IRON_LAUNCH((gqa_decode_kernel<4>), grid, block, 0, s, a);
      IRON_LAUNCH((gqa_combine_kernel<4>), cgrid, cblock, 0, s, a);
      break;
    default:
      IRON_LAUNCH((gqa_decode_kernel<8>), grid, block, 0, s, a);
      IRON_LAUNCH((gqa_combine_kernel<8>), cgrid, cblock, 0, s, a);
      break;
  }
  return check_launch(who);
}

extern "C" int iron_gqa_decode(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                               const float* angles, int angle_rows, void* out, void* workspace, int n_heads,
                               int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev, float scale,
                               void* stream) {
  return gqa_decode_launch("iron_gqa_decode", q, k_new, v_new, k_cache, v_cache, angles, angle_rows, out, workspace,
                           n_heads, n_kv_heads, head_dim, max_len, pos, pos_dev, scale, stream);
}

// The workspace of iron_gqa_decode_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends. Host code never passes `scratch`
// itself to a kernel (on the host that name is a stand-in, not a device
// address): its device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and only that address is used.
static constexpr long long kDecodeScratchBytes = 4LL << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device (looked up on the first
// call per device), or nullptr with the error set.
static void* decode_scratch_ptr(const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("%s: device %d beyond the %d devices the library tracks", who, dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", who, dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

extern "C" long long iron_gqa_decode_noalloc_max_bytes(void) { return kDecodeScratchBytes; }

extern "C" int iron_gqa_decode_noalloc(const void* q, const void* k_new, const void* v_new, void* k_cache,
                                       void* v_cache, const float* angles, int angle_rows, void* out, int n_heads,
                                       int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev,
                                       float scale, void* stream) {
  const long long need = iron_gqa_decode_workspace_bytes(n_heads, n_kv_heads, head_dim, max_len);
  IRON_REQUIRE(need > 0, "iron_gqa_decode_noalloc: invalid shape (n_heads=%d, n_kv_heads=%d, head_dim=%d, max_len=%d)",
               n_heads, n_kv_heads, head_dim, max_len);
  IRON_REQUIRE(need <= kDecodeScratchBytes,
               "iron_gqa_decode_noalloc: this shape needs %lld bytes of scratch, more than the %lld the library "
               "holds per device (use iron_gqa_decode with a workspace)", need, kDecodeScratchBytes);
  void* ws = decode_scratch_ptr("iron_gqa_decode_noalloc");
  if (!ws) return IRON_EINVAL;
  return gqa_decode_launch("iron_gqa_decode_noalloc", q, k_new, v_new, k_cache, v_cache, angles, angle_rows, out, ws,
                           n_heads, n_kv_heads, head_dim, max_len, pos, pos_dev, scale, stream);
}

extern "C" int iron_attention_prefill(const void* q, const void* k, const void* v, void* out, int n_heads,
                                      int n_kv_heads, int seq_q, int seq_kv, int head_dim, long long q_head_stride,
                                      long long q_row_stride, long long kv_head_stride, long long kv_row_stride,
                                      long long o_head_stride, long long o_row_stride, int out_rows, int causal,
                                      int q_offset, float scale, void* stream) {
  IRON_REQUIRE(q && k && v && out, "iron_attention_prefill: null pointer");
  IRON_REQUIRE(head_dim == kD, "iron_attention_prefill: head_dim=%d (only 64 is supported)", head_dim);
  IRON_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "iron_attention_prefill: n_heads=%d must be a multiple of n_kv_heads=%d", n_heads, n_kv_heads);
  IRON_REQUIRE(seq_q > 0 && seq_kv > 0, "iron_attention_prefill: empty sequence");
  IRON_REQUIRE(q_offset >= 0, "iron_attention_prefill: q_offset must be >= 0");
  IRON_REQUIRE(scale > 0.f && scale < INFINITY, "iron_attention_prefill: scale=%g must be positive and finite",
               static_cast<double>(scale));
  if (out_rows < seq_q) out_rows = seq_q;
  IRON_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && q_row_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                   kv_row_stride % 8 == 0 && kv_head_stride % 8 == 0,
               "iron_attention_prefill: rows must be 16-byte aligned");
  PrefillArgs a{static_cast<const uint16_t*>(q),
                static_cast<const uint16_t*>(k),
                static_cast<const uint16_t*>(v),
                static_cast<uint16_t*>(out),
                q_head_stride,
                q_row_stride,
                kv_head_stride,
                kv_row_stride,
                kv_head_stride,
                kv_row_stride,
                o_head_stride,
                o_row_stride,
                n_heads,
                n_kv_heads,
                seq_q,
                seq_kv,
                out_rows,
                causal,
                q_offset,
                scale * 1.4426950408889634f};
  IRON_REQUIRE(aligned16(out) && o_row_stride % 8 == 0 && o_head_stride % 8 == 0,
               "iron_attention_prefill: out rows must be 16-byte aligned");
  IRON_REQUIRE((out_rows + kFaQ - 1) / kFaQ < 65536, "iron_attention_prefill: out_rows=%d too large", out_rows);
  dim3 grid(n_heads, (out_rows + kFaQ - 1) / kFaQ), block(256);
  IRON_LAUNCH(attention_prefill_kernel, grid, block, 0, static_cast<hipStream_t>(stream), a);
  return check_launch("attention_prefill");
}
