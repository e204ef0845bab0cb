// GQA attention for decode (split-K flash-decode) and causal prefill.
//
// Decode: one new token. A workgroup owns (KV head j, a chunk of 64 cache
// positions) and serves the G = H/Hkv query heads that share KV head j, so
// every K/V byte is read from HBM once for all of them. Inside the chunk the
// scores (K Q^T) and the output (P V) run on the matrix cores, the softmax in
// fp32 (scores scaled by log2(e)/sqrt(D), exp2); the chunk's unnormalised
// output, maximum and sum go to a workspace and are merged over the chunks.
// When Hkv is a multiple of 8 the merge happens in the same launch: all
// chunks of one KV head run on one XCD (workgroups are dispatched to the 8
// XCDs round-robin), so their partials meet in that XCD's L2, and the last
// workgroup of the head to count itself in (an atomic in that L2) merges them.
// A merge across XCDs in one launch was measured slower than a second launch:
// it needs an agent-scope release (a write-back of the whole per-XCD L2,
// serialised across workgroups) or write-through stores and device-scope
// atomics. Other Hkv use a second small kernel for the merge.
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
  float* part;            // per KV head (head_stride floats): nsplit partials of part_stride<G>() floats
  unsigned* ctr;          // per KV head (kCtrStride words): arrival counter of the one-launch path
  long long head_stride;  // floats between the partial regions of consecutive KV heads
  const int* pos_dev;     // optional device-resident position (overrides pos)
  int pos;
  int max_len;
  int angle_rows;
  int nsplit;             // chunks per KV head
  float scale_log2;       // log2(e) * scale
};

// One chunk's partial: G x 64 unnormalised outputs, then G maxima, then G
// sums, padded to a whole number of 16-byte quads.
template <int G>
constexpr int part_stride() {
  return (G * kD + 2 * G + 3) / 4 * 4;
}

// Workgroups are dispatched to the XCDs round-robin, so workgroups whose
// linear ids agree mod 8 run on one XCD and share its L2. The one-launch path
// gives each KV head such a class of ids (n_kv_heads a multiple of 8).
constexpr int kXcds = 8;
constexpr int kCtrStride = 32;  // counter words per KV head: one 128-byte line each

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

// Cross-lane exchanges by v_permlane32_swap_b32 / v_permlane16_swap_b32 with
// both operands holding a: afterwards x[l] = a[l % 32], y[l] = a[l % 32 + 32]
// (split32), or x[l], y[l] = a of the even and odd 16-lane row of l's pair
// (split16), so that op(x, y) = op(a[l], a[l ^ 32]) (resp. a[l ^ 16]) on
// every lane. Inline assembly: this compiler's builtins for the permlane swaps
// return the first result in place of the second (seen in the generated code).
// The s_nop covers the VALU-write to permlane-read hazard.
__device__ __forceinline__ void split32(float a, float& x, float& y) {
  unsigned u = __builtin_bit_cast(unsigned, a), v = u;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(v));
  x = __builtin_bit_cast(float, u);
  y = __builtin_bit_cast(float, v);
}
__device__ __forceinline__ void split16(float a, float& x, float& y) {
  unsigned u = __builtin_bit_cast(unsigned, a), v = u;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(u), "+v"(v));
  x = __builtin_bit_cast(float, u);
  y = __builtin_bit_cast(float, v);
}
// max / sum over lanes {l, l ^ 16, l ^ 32, l ^ 48}
__device__ __forceinline__ float max_over_rows(float a) {
  float x, y;
  split32(a, x, y);
  a = fmaxf(x, y);
  split16(a, x, y);
  return fmaxf(x, y);
}
__device__ __forceinline__ float sum_over_rows(float a) {
  float x, y;
  split32(a, x, y);
  a = x + y;
  split16(a, x, y);
  return x + y;
}

// 2^x by v_exp_f32 alone, for x <= 0 (softmax weights): results below 2^-126
// flush to zero, which the weights tolerate; elsewhere exp2f's value.
__device__ __forceinline__ float exp2_weight(float x) { return __builtin_amdgcn_exp2f(x); }

typedef __bf16 dec_bf16x8 __attribute__((ext_vector_type(8)));
typedef short dec_i16x4 __attribute__((ext_vector_type(4)));
typedef float dec_f32x4 __attribute__((ext_vector_type(4)));

// Slot of 16-byte chunk c of V row R (0..15) in a wave's LDS block: rows of
// one parity in a 32-lane pass of the transposed read (R, R + 2, R + 4, R + 6)
// land on disjoint bank groups. An involution in c.
__device__ __forceinline__ int dec_v_slot(int R, int c) { return c ^ (((R >> 1) & 3) << 1); }

// One decode step of KV head j for its G query heads; workgroup s owns cache
// positions [64 s, 64 s + 64), wave w of it positions 64 s + 16 w + [0, 16).
//
// Per wave, on the matrix cores (v_mfma_f32_16x16x32_bf16 for the scores,
// v_mfma_f32_16x16x16_bf16 for the output):
//   S = K Q^T    A = the wave's 16 K rows straight from global memory (lane l:
//                row l % 16, dims 8 (l / 16) + [0, 8) and 32 + the same),
//                B = rotated q from LDS (column = head l % 16; heads >= G
//                repeat a real head, and their rows of P and O are dropped);
//                lane l then holds the scores of head l % 16 at positions
//                4 (l / 16) + [0, 4).
//   softmax      per head over the wave's 16 positions: the lane's own 4
//                values and two permlane exchanges; fp32 weights in the log2
//                domain.
//   O = P V      A = P as bf16 pairs hi + lo (two MFMAs: the weights keep
//                ~16 bits), B = V^T read from the wave's LDS block (the V rows,
//                loaded to registers, stored there) with ds_read_b64_tr_b16; lane l (l / 16 <
//                G / 4) ends with heads 4 (l / 16) + [0, 4) at dims 16 t + l % 16.
// The new token's k (rotated) and v replace their row (and are appended to
// the caches); rows past pos are masked (scores) and zeroed (V). The four
// waves' (max, sum, output) meet once in LDS to form the chunk's partial.
//
// MERGE (the one-launch path): workgroup n takes KV head 8 (t / nsplit) + n % 8
// and chunk t % nsplit, t = n / 8, so all chunks of a head run on one XCD.
// After writing its partial a workgroup waits for its stores to reach that
// XCD's L2 and counts itself in with an atomic there; the last of the head's
// active chunks to arrive invalidates its CU's L1 and merges the head's
// partials from the L2 (fused_merge), then returns the counter to zero. No
// workgroup waits for another. Without MERGE the grid is (nsplit, Hkv) and
// gqa_combine_kernel merges.
template <int G>
__device__ void fused_merge(const DecodeArgs& a, int j, int nact, int tid);

template <int G, bool MERGE, bool RES>
__global__ __launch_bounds__(kDecThreads) void gqa_decode_kernel(DecodeArgs a) {
  constexpr int D = kD;
  constexpr int NW = kDecThreads / kWave;
  constexpr int PS = part_stride<G>();
  __shared__ __attribute__((aligned(16))) uint16_t q_s[G * D];  // rotated q, bf16
  __shared__ float wm_s[NW][G], wl_s[NW][G];
  __shared__ __attribute__((aligned(16))) float wo_s[NW][G * D];
  __shared__ __attribute__((aligned(16))) unsigned char v_s[NW][16 * 128];  // each wave's 16 V rows

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid >> 6;
  int s, j;
  if constexpr (MERGE) {
    const int n = blockIdx.x, t = n / kXcds;
    j = n % kXcds + kXcds * (t / a.nsplit);
    s = t % a.nsplit;
  } else {
    s = blockIdx.x;
    j = blockIdx.y;
  }
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  if (pos < 0 || pos >= a.max_len || pos >= a.angle_rows) return;  // rejected on the host when pos is known
  const int L = pos + 1;
  const int p0 = s * kDecChunk;
  if (p0 >= L) return;
  const int r = lane & 15, cq = lane >> 4;
  const int wrow0 = p0 + 16 * w;
  const bool owner_wave = pos >= wrow0 && pos < wrow0 + 16;
  const bool owner = pos == wrow0 + r;  // the 4 lanes holding the new token's K row
  const size_t hb = static_cast<size_t>(j) * a.max_len;

  // Loads, oldest first: the new token's table entries and k/v (owner lanes),
  // then q and its table row, then the K rows, then the V rows. q is rotated
  // while K and V are still in flight (the waits below count only what the
  // rotation needs), and the scores wait for K alone.
  const float* angrow = a.angles + static_cast<size_t>(pos) * D;
  float ang[16];
  uint4 kna = make_uint4(0, 0, 0, 0), knb = kna, vna = kna, vnb = kna;
  if (owner) {  // the new token's table entries (dims 8 cq + [0, 8)) and k/v chunks cq, cq + 4
    const float4* ap = reinterpret_cast<const float4*>(angrow + cq * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 t = ap[i];
      ang[4 * i] = t.x;
      ang[4 * i + 1] = t.y;
      ang[4 * i + 2] = t.z;
      ang[4 * i + 3] = t.w;
    }
    kna = *reinterpret_cast<const uint4*>(a.k_new + static_cast<size_t>(j) * D + cq * 8);
    knb = *reinterpret_cast<const uint4*>(a.k_new + static_cast<size_t>(j) * D + (cq + 4) * 8);
    vna = *reinterpret_cast<const uint4*>(a.v_new + static_cast<size_t>(j) * D + cq * 8);
    vnb = *reinterpret_cast<const uint4*>(a.v_new + static_cast<size_t>(j) * D + (cq + 4) * 8);
  }
  constexpr int QN = (G * D + kDecThreads - 1) / kDecThreads;  // q elements per thread
  const uint16_t* qh = a.q + static_cast<size_t>(j) * G * D;
  uint16_t qx[QN], qp[QN];
  float2 qa[QN];
#pragma unroll
  for (int e = 0; e < QN; ++e) {
    const int t = min(tid + kDecThreads * e, G * D - 1), i = (t % D) & 31;
    qx[e] = qh[t];
    qp[e] = qh[t ^ 32];
    qa[e] = *reinterpret_cast<const float2*>(angrow + 2 * i);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the q loads ahead of the K/V loads
  // K rows (clamped: rows >= pos are replaced or masked below). RES: the caches
  // stay resident between calls (a decode loop over all layers; ~134 MB at 4096
  // positions fits the Infinity Cache while the weights stream past it), so the
  // K/V loads are ordinary, allocating loads (decode +0.9%). Otherwise they are
  // streaming loads, faster when the caches come from HBM every time.
  auto ld_kv = [](const uint16_t* p) { return RES ? *reinterpret_cast<const uint4*>(p) : ld_stream16(p); };
  const int krow = min(wrow0 + r, a.max_len - 1);
  uint4 k0 = ld_kv(a.k_cache + (hb + krow) * D + cq * 8);
  uint4 k1 = ld_kv(a.k_cache + (hb + krow) * D + (cq + 4) * 8);
  // V rows: lane l of load u holds row 8 u + l / 8, 16-byte chunk dec_v_slot(row, l % 8),
  // stored below into slot l % 8 of the wave's LDS block
  unsigned char* vblk = v_s[w];
  uint4 vraw[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int R = 8 * u + (lane >> 3);
    const int vrow = min(wrow0 + R, a.max_len - 1);
    vraw[u] = ld_kv(a.v_cache + (hb + vrow) * D + dec_v_slot(R, lane & 7) * 8);
  }
#pragma unroll
  for (int e = 0; e < QN; ++e) {
    const int t = tid + kDecThreads * e;
    if (t < G * D) {
      const float x = bf16_to_f32(qx[e]), xp = bf16_to_f32(qp[e]);
      q_s[t] = f32_to_bf16((t % D) < 32 ? x * qa[e].x - xp * qa[e].y : x * qa[e].x + xp * qa[e].y);
    }
  }
  // barrier without a wait for the K/V loads in flight (__syncthreads would
  // wait for all of them); the memory clobber keeps the q_s accesses on their sides
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const int hq = r & (G - 1);
  const dec_bf16x8 qb0 = *reinterpret_cast<const dec_bf16x8*>(&q_s[hq * D + cq * 8]);
  const dec_bf16x8 qb1 = *reinterpret_cast<const dec_bf16x8*>(&q_s[hq * D + (cq + 4) * 8]);

  if (owner) {  // rotate the new k, append k/v to the caches
    float lo[8], hi[8];
    rope_chunk(kna, knb, ang, true, lo);
    rope_chunk(knb, kna, ang, false, hi);
    k0 = make_uint4(pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3]), pack_bf16x2(lo[4], lo[5]),
                    pack_bf16x2(lo[6], lo[7]));  // exact: bf16 values
    k1 = make_uint4(pack_bf16x2(hi[0], hi[1]), pack_bf16x2(hi[2], hi[3]), pack_bf16x2(hi[4], hi[5]),
                    pack_bf16x2(hi[6], hi[7]));
    uint16_t* kp = a.k_cache + (hb + pos) * D;
    uint16_t* vp = a.v_cache + (hb + pos) * D;
    *reinterpret_cast<uint4*>(kp + cq * 8) = k0;
    *reinterpret_cast<uint4*>(kp + (cq + 4) * 8) = k1;
    *reinterpret_cast<uint4*>(vp + cq * 8) = vna;
    *reinterpret_cast<uint4*>(vp + (cq + 4) * 8) = vnb;
  }

  // One code path for waves whose 16 rows are all valid and none is the new
  // token (every wave but the last one or two), one with the masks and the
  // owner's row.
  const bool full = wrow0 + 16 <= L && !owner_wave;  // wave-uniform
  auto wave_body = [&](auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    dec_f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
    sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dec_bf16x8, k0), qb0, sacc, 0, 0, 0);
    sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dec_bf16x8, k1), qb1, sacc, 0, 0, 0);

    // softmax of head r over positions wrow0 + 4 cq + i (log2 domain)
    float sv[4];
    bool valid[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      valid[i] = FULL || wrow0 + 4 * cq + i < L;
      sv[i] = valid[i] ? sacc[i] * a.scale_log2 : -INFINITY;
    }
    const float m = max_over_rows(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));  // -inf only if all 16 rows are past pos
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = FULL || valid[i] ? exp2_weight(sv[i] - m) : 0.f;
    const float lsum = sum_over_rows((e[0] + e[1]) + (e[2] + e[3]));
    // P = hi + lo, both bf16
    const uint32_t h01 = pack_bf16x2(e[0], e[1]), h23 = pack_bf16x2(e[2], e[3]);
    const uint32_t l01 = pack_bf16x2(e[0] - lo_bf16(h01), e[1] - hi_bf16(h01));
    const uint32_t l23 = pack_bf16x2(e[2] - lo_bf16(h23), e[3] - hi_bf16(h23));
    const dec_i16x4 phi = __builtin_bit_cast(dec_i16x4, make_uint2(h01, h23));
    const dec_i16x4 plo = __builtin_bit_cast(dec_i16x4, make_uint2(l01, l23));

    // V rows into the wave's LDS block; rows past pos become zeros (0 x stale
    // data must not reach O), the new token's row takes v_new
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bool stale = !FULL && wrow0 + 8 * u + (lane >> 3) > pos;
      *reinterpret_cast<uint4*>(vblk + u * 1024 + lane * 16) = stale ? make_uint4(0, 0, 0, 0) : vraw[u];
    }
    if (!FULL && owner) {
      *reinterpret_cast<uint4*>(vblk + r * 128 + dec_v_slot(r, cq) * 16) = vna;
      *reinterpret_cast<uint4*>(vblk + r * 128 + dec_v_slot(r, cq + 4) * 16) = vnb;
    }
    // V^T operands: in each 16-lane group g lane 4 jj + qq addresses row 4 g + jj,
    // dims 16 t + 4 qq .. + 3; lane i of the group then receives dim 16 t + i
    // of rows 4 g + [0, 4)
    const int tR = 4 * cq + (r >> 2);
    const unsigned vb = static_cast<unsigned>(reinterpret_cast<uintptr_t>(vblk)) + tR * 128 + 8 * (lane & 1);
    uint2 vt[4];
    {
      unsigned ad[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) ad[t] = vb + dec_v_slot(tR, 2 * t + ((lane & 3) >> 1)) * 16;
      asm volatile(
          "ds_read_b64_tr_b16 %0, %4\n\tds_read_b64_tr_b16 %1, %5\n\t"
          "ds_read_b64_tr_b16 %2, %6\n\tds_read_b64_tr_b16 %3, %7\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(vt[0]), "=&v"(vt[1]), "=&v"(vt[2]), "=&v"(vt[3])
          : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3])
          : "memory");
    }
    dec_f32x4 o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const dec_i16x4 vv = __builtin_bit_cast(dec_i16x4, vt[t]);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(phi, vv, dec_f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(plo, vv, o[t], 0, 0, 0);
    }
    if (lane < G) {
      wm_s[w][lane] = m;
      wl_s[w][lane] = lsum;
    }
    if (4 * cq < G) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * cq + i < G) wo_s[w][(4 * cq + i) * D + 16 * t + r] = o[t][i];
    }
  };
  if (full)
    wave_body(std::true_type{});
  else
    wave_body(std::false_type{});
  __syncthreads();

  // the chunk's partial: the four waves merged
  float* part = a.part + static_cast<size_t>(j) * a.head_stride + static_cast<size_t>(s) * PS;
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
  if constexpr (MERGE) {
    __shared__ int last_s;
    const int nact = (L + kDecChunk - 1) / kDecChunk;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores have reached the L2
    __syncthreads();
    if (tid == 0) {
      unsigned* c = a.ctr + static_cast<size_t>(j) * kCtrStride;
      const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      const int last = old == static_cast<unsigned>(nact - 1);
      if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      last_s = last;
    }
    __syncthreads();
    if (!last_s) return;
    asm volatile("buffer_inv sc0" ::: "memory");  // no stale line of the head's partials in this CU's L1
    fused_merge<G>(a, j, nact, tid);
  }
}

// The merge of KV head j's nact chunk partials by one 256-thread workgroup,
// in batches of 64 chunks. Per batch, the statistics first: one wave per
// head takes the batch's 64 maxima (a DPP reduction), raises the head's
// running maximum, and leaves each chunk's weight exp2(M_c - M) in LDS, with
// the running sum and the factor that rescales the earlier batches. Then the
// outputs: thread -> 4 consecutive values (quad qd of the G x 64) and slice q
// of the chunks (c0 + q + NQ b), its weights read as one vector from LDS, one
// FMA per value and chunk. The loads of the statistics and of the outputs are
// all issued before the statistics are used (one round trip); chunks past
// nact load chunk nact - 1 and weigh 0, and the number of output loads per
// thread is the live count rounded up to 4, 8 or 16. The NQ slices meet in LDS
// at the end. Every sum runs in a fixed order: the result depends only on the
// data.
template <int G>
__device__ void fused_merge(const DecodeArgs& a, int j, int nact, int tid) {
  constexpr int D = kD;
  constexpr int PS = part_stride<G>();
  constexpr int CB = 64;                      // chunks per batch
  constexpr int NQD = G * D / 4;              // output quads per chunk
  constexpr int NQ = kDecThreads / NQD;       // chunk slices
  constexpr int PER = CB / NQ;                // chunks per thread per batch
  constexpr int NE = (CB * G + kDecThreads - 1) / kDecThreads;  // (head, chunk) pairs per thread
  __shared__ __attribute__((aligned(16))) float w_s[G * CB];    // [head][slice][b]
  __shared__ float mh_s[G], lh_s[G], sc_s[G];
  __shared__ float4 oo_s[kDecThreads];
  const int lane = tid & (kWave - 1);
  const int qd = tid % NQD, q = tid / NQD, g = qd / (D / 4);
  const float* base = a.part + static_cast<size_t>(j) * a.head_stride;
  if (tid < G) {
    mh_s[tid] = -INFINITY;
    lh_s[tid] = 0.f;
  }
  __syncthreads();
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  auto load_o = [&](int c0, int b) {
    return *reinterpret_cast<const float4*>(base + static_cast<size_t>(min(c0 + q + NQ * b, nact - 1)) * PS + 4 * qd);
  };
  // one batch with N (<= 16) output loads per thread per round
  auto batch = [&](auto n_tag, int c0) {
    constexpr int N = decltype(n_tag)::value;
    float st_m[NE], st_l[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int p = tid + kDecThreads * e, h = min(p / CB, G - 1), c = c0 + p % CB;
      const float* pk = base + static_cast<size_t>(min(c, nact - 1)) * PS;
      st_m[e] = pk[G * D + h];
      st_l[e] = pk[G * D + G + h];
    }
    __builtin_amdgcn_sched_barrier(0);  // statistics first: their wait leaves the output loads in flight
    float4 ob[N];
#pragma unroll
    for (int b = 0; b < N; ++b) ob[b] = load_o(c0, b);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int p = tid + kDecThreads * e;
      if (p < CB * G) {  // whole waves: one head each
        const int h = p / CB, cb = p % CB;
        const bool live = c0 + cb < nact;
        const float m = live ? st_m[e] : -INFINITY;
        const float mb = wave_max(m);  // finite: chunk c0 is live
        const float mo = mh_s[h];
        const float mn = fmaxf(mo, mb);
        const float wgt = exp2_weight(m - mn);  // 0 past nact
        w_s[(h * NQ + cb % NQ) * PER + cb / NQ] = wgt;
        const float ls = wave_sum(live ? wgt * st_l[e] : 0.f);
        if (lane == 0) {
          const float sc = exp2_weight(mo - mn);  // 0 on the first batch
          sc_s[h] = sc;
          mh_s[h] = mn;
          lh_s[h] = fmaf(lh_s[h], sc, ls);
        }
      }
    }
    __syncthreads();
    const float sc = sc_s[g];
    acc.x *= sc;
    acc.y *= sc;
    acc.z *= sc;
    acc.w *= sc;
    const float* wrow = &w_s[(g * NQ + q) * PER];
#pragma unroll
    for (int b0 = 0; b0 < PER; b0 += N) {
      if (b0 > 0) {
        if (c0 + q + NQ * b0 >= nact) break;  // no live chunk left in this slice
#pragma unroll
        for (int b = 0; b < N; ++b) ob[b] = load_o(c0, b0 + b);
      }
      float wv[N];
#pragma unroll
      for (int b = 0; b < N; b += 4) {
        const float4 t = *reinterpret_cast<const float4*>(wrow + b0 + b);
        wv[b] = t.x;
        wv[b + 1] = t.y;
        wv[b + 2] = t.z;
        wv[b + 3] = t.w;
      }
#pragma unroll
      for (int b = 0; b < N; ++b) {
        acc.x = fmaf(wv[b], ob[b].x, acc.x);
        acc.y = fmaf(wv[b], ob[b].y, acc.y);
        acc.z = fmaf(wv[b], ob[b].z, acc.z);
        acc.w = fmaf(wv[b], ob[b].w, acc.w);
      }
      if (N < PER && b0 + N >= PER) break;
      if (N < 16) break;  // a short batch takes one round
    }
    __syncthreads();  // w_s and sc_s are rewritten by the next batch
  };
  for (int c0 = 0; c0 < nact; c0 += CB) {
    const int span = (min(CB, nact - c0) + NQ - 1) / NQ;  // live chunks per slice (uniform)
    if (span <= 4 && PER >= 4)
      batch(std::integral_constant<int, (PER < 4 ? PER : 4)>{}, c0);
    else if (span <= 8 && PER >= 8)
      batch(std::integral_constant<int, 8>{}, c0);
    else
      batch(std::integral_constant<int, (PER < 16 ? PER : 16)>{}, c0);
  }
  oo_s[tid] = acc;
  __syncthreads();
  if (q == 0) {
    float4 ot = acc;
#pragma unroll
    for (int qq = 1; qq < NQ; ++qq) {
      const float4 o = oo_s[qq * NQD + qd];
      ot.x += o.x;
      ot.y += o.y;
      ot.z += o.z;
      ot.w += o.w;
    }
    const float rl = __builtin_amdgcn_rcpf(lh_s[g]);
    const uint32_t lo = cvt_pk_bf16(ot.x * rl, ot.y * rl), hi = cvt_pk_bf16(ot.z * rl, ot.w * rl);
    *reinterpret_cast<uint2*>(a.out + static_cast<size_t>(j) * G * D + 4 * qd) = make_uint2(lo, hi);
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
  const float* base = a.part + static_cast<size_t>(j) * a.head_stride;
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

// Zeroes the arrival counters of the one-launch path (one word per KV head),
// for callers whose workspace carries no state between calls.
__global__ __launch_bounds__(kWave) void gqa_clear_counters_kernel(unsigned* ctr, int n_kv_heads) {
  for (int j = threadIdx.x; j < n_kv_heads; j += kWave) ctr[static_cast<size_t>(j) * kCtrStride] = 0u;
}

// ---------------------------------------------------------------------------
// Prefill / MHA: causal (optional) flash attention over strided Q, K, V on
// MFMA (v_mfma_f32_32x32x16_bf16).
//
// Workgroup = 4 waves = 128 queries of one head; each wave owns 32 queries and
// walks the visible keys in blocks of 64. K and V blocks are staged row-major
// in a 4-stage LDS ring filled by LDS-direct loads (buffer_load_dwordx4 ... lds,
// load_lds16: no VGPR staging, no LDS stores), up to three blocks ahead of the
// one being computed, one barrier per block. Per block a wave computes S^T = K Q^T (two 32x32 tiles): every lane
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
  // Use the Q fragments here, before any K/V load is issued: the compiler then
  // waits for these four loads now. Otherwise it counts them as outstanding at
  // their first use inside the key loop and waits there with vmcnt, which also
  // drains the K/V blocks the loop keeps in flight (the compiler does not count
  // those assembly loads).
  asm volatile("" ::"v"(qf[0]), "v"(qf[1]), "v"(qf[2]), "v"(qf[3]));
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
  // Blocks are issued in order 0, 1, 2, ...: each lane keeps the byte offset of
  // its next row (from the head's K or V base, through a buffer resource: see
  // load_lds16) and bumps it by 64 rows per issue; only a block that runs past
  // Skv recomputes clamped offsets.
  const i32x4v rsrc_k = buffer_rsrc(a.k + hk * a.k_hs), rsrc_v = buffer_rsrc(a.v + hk * a.v_hs);
  unsigned coff[4], rsb[4], next_off[4];
  int lrow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = wave * 4 + j;
    const bool is_k = b < 8;
    const int r = (b & 7) * 8 + (lane >> 3), slot = lane & 7;
    const int chunk = is_k ? fa_k_slot(r, slot) : fa_v_slot(r, slot);  // both are involutions
    coff[j] = chunk * 16;
    rsb[j] = static_cast<unsigned>((is_k ? a.k_rs : a.v_rs) * 2);
    lrow[j] = r;
    next_off[j] = coff[j] + r * rsb[j];
  }
  auto issue = [&](int bi) {
    unsigned char* st = lds + (bi % kFaStages) * 2 * kFaBlock;
    const bool inside = bi * kFaK + kFaK <= a.Skv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned off = inside ? next_off[j] : coff[j] + min(bi * kFaK + lrow[j], a.Skv - 1) * rsb[j];
      load_lds16(wave * 4 + j < 8 ? rsrc_k : rsrc_v, off, st + (wave * 4 + j) * 1024);
      next_off[j] += kFaK * rsb[j];
    }
  };
  // this lane's transposed-read address inside a V block: 16-lane group g
  // covers dims 16 (g % 2) .. + 15 (+ 32 db) and keys 4 hh .. + 3 (+ 16 st, + 8)
  const int tr_row = 4 * hh + ((lane & 15) >> 2), tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // S^T = K Q^T for block bi: sc[b][j] is key 64 bi + 32 b + 8 (j / 4) + 4 hh + j % 4, query qw + c.
  // k_frags reads the block's K fragments (A operand: key 32 b + c, dims 16 kk + 8 hh .. + 8);
  // s_mfma runs the two independent accumulation chains (b = 0, 1) interleaved.
  auto k_frags = [&](int bi, fa_bf16x8 (&kf)[2][4]) {
    const unsigned char* ks = lds + (bi % kFaStages) * 2 * kFaBlock;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int kr = 32 * b + c;
        kf[b][kk] = __builtin_bit_cast(
            fa_bf16x8, *reinterpret_cast<const fa_u32x4*>(ks + kr * 128 + fa_k_slot(kr, 2 * kk + hh) * 16));
      }
  };
  auto s_mfma = [&](const fa_bf16x8 (&kf)[2][4], fa_f32x16 (&sc)[2]) {
    fa_f32x16 acc0 = {}, acc1 = {};  // the first MFMAs take an inline zero accumulator
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[0][kk], qf[kk], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[1][kk], qf[kk], acc1, 0, 0, 0);
    }
    sc[0] = acc0;
    sc[1] = acc1;
  };
  auto scores = [&](int bi, fa_f32x16 (&sc)[2]) {
    fa_bf16x8 kf[2][4];
    k_frags(bi, kf);
    s_mfma(kf, sc);
  };
  auto visible = [&](int bi) { return !a.causal || bi * kFaK <= wave_last; };

  // Software pipeline over key blocks: iteration bi waits for block bi+1 and
  // reads its K fragments and block bi's V^T fragments, takes block bi's row
  // maximum, then runs block bi+1's S^T MFMAs, block bi's exponentials and its
  // P V MFMAs in one branch-free stretch, so that the matrix cores work while
  // the softmax occupies the VALU. Stages: bi (V being read), bi+1 (K being
  // read), bi+2 in flight, bi+3 being issued into the stage block bi-1 used.
  // On the last iteration the K fragments come from a stage no load writes any
  // more and the scores they give are not used.
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
  scores(0, sa);  // block 0 is visible to every wave

  auto step = [&](int bi, fa_f32x16 (&cur)[2], fa_f32x16 (&nxt)[2]) {
    if (bi + 1 < nb) {
      if (bi + 2 < nb)
        fa_wait_loads_barrier<4>();
      else
        fa_wait_loads_barrier<0>();
      // block bi-1's stage is free: every wave passed this barrier after its last read of it
      if (bi + kFaStages - 1 < nb) issue(bi + kFaStages - 1);
    }
    if (!visible(bi)) return;  // every key of the block (and of the next) is after this wave's queries
    fa_bf16x8 kf[2][4];
    k_frags(bi + 1, kf);  // issued now; the compiler waits for them (exact LDS counts) before their MFMAs
    const int k0 = bi * kFaK;
    const unsigned char* vs = lds + (bi % kFaStages) * 2 * kFaBlock + kFaBlock;
      // V^T fragments for O^T += V^T P^T: k-step st, element i of lane (d, hh) is
      // key 16 st + 8 (i / 4) + 4 hh + i % 4 (two transposed reads of 4 keys each).
      // The address of (st, hl) is the (0, 0) one plus 2048 st + 1024 hl: the
      // swizzle (fa_v_slot) depends on bit 1 of the row only, which st and hl do
      // not change, so those steps become the reads' immediate offsets. As
      // builtins the reads get exact LDS waits (the K/V loads are assembly the
      // compiler does not count), so it can issue them early and wait only
      // before the P V MFMAs.
      fa_u32x2 vt[2][4][2];
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const int dim = 32 * db + tr_dim;
        const unsigned char* vb = vs + tr_row * 128 + fa_v_slot(tr_row, dim >> 3) * 16 + (dim & 7) * 2;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int hl = 0; hl < 2; ++hl)
            vt[db][st][hl] = __builtin_bit_cast(
                fa_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                              (__attribute__((address_space(3))) fa_i16x4*)(vb + 2048 * st + 1024 * hl)));
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
        mx = fmaxf(fmaxf(cur[0][0], cur[0][1]), cur[0][2]);  // a chain of v_max3_f32
#pragma unroll
        for (int j = 3; j < 15; j += 2) mx = fmaxf(fmaxf(mx, cur[0][j]), cur[0][j + 1]);
        mx = fmaxf(fmaxf(mx, cur[0][15]), cur[1][0]);
#pragma unroll
        for (int j = 1; j < 15; j += 2) mx = fmaxf(fmaxf(mx, cur[1][j]), cur[1][j + 1]);
        mx = fmaxf(mx, cur[1][15]);
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
      s_mfma(kf, nxt);  // block bi+1's scores, independent of everything below
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

static int decode_part_stride(int G) {
  switch (G) {
    case 1: return part_stride<1>();
    case 2: return part_stride<2>();
    case 4: return part_stride<4>();
    default: return part_stride<8>();
  }
}

// Workspace layout: the arrival counters (one 128-byte line per KV head,
// rounded up to 256 bytes), then per KV head its nsplit chunk partials,
// each head's region rounded up to 256 bytes.
static long long decode_ctr_bytes(int n_kv_heads) { return (static_cast<long long>(n_kv_heads) * kCtrStride * 4 + 255) / 256 * 256; }
static long long decode_head_stride(int G, int max_len) {
  return (static_cast<long long>(decode_nsplit(max_len)) * decode_part_stride(G) + 63) / 64 * 64;
}

extern "C" long long iron_gqa_decode_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int max_len) {
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim != kD || max_len <= 0) return -1;
  const int G = n_heads / n_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return -1;
  return decode_ctr_bytes(n_kv_heads) + static_cast<long long>(n_kv_heads) * decode_head_stride(G, max_len) * 4;
}

// Checks and launches of one GQA decode step with its counters and partials
// in `workspace` (iron_gqa_decode_workspace_bytes() of the shape, 256-byte
// aligned); shared by the entry point that takes a workspace (counters kept
// at zero between calls) and the one that uses the library's own scratch
// array (clear_counters: zeroed before each call by a small kernel).
// One launch (n_kv_heads a multiple of 8: each KV head's chunks on one XCD,
// merged by the last to finish) or the partials kernel plus the merge kernel.
template <int G, bool RES>
static void gqa_decode_dispatch(const DecodeArgs& a, int n_kv_heads, hipStream_t s) {
  const dim3 block(kDecThreads);
  if (n_kv_heads % kXcds == 0) {
    IRON_LAUNCH((gqa_decode_kernel<G, true, RES>), dim3(a.nsplit * n_kv_heads), block, 0, s, a);
  } else {
    IRON_LAUNCH((gqa_decode_kernel<G, false, RES>), dim3(a.nsplit, n_kv_heads), block, 0, s, a);
    IRON_LAUNCH((gqa_combine_kernel<G>), dim3(n_kv_heads * G), dim3(kMergeThreads), 0, s, a);
  }
}

static int gqa_decode_launch(const char* who, const void* q, const void* k_new, const void* v_new, void* k_cache,
                             void* v_cache, const float* angles, int angle_rows, void* out, void* workspace,
                             int n_heads, int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev,
                             float scale, void* stream, bool clear_counters, int flags) {
  IRON_REQUIRE((flags & ~IRON_GQA_KV_RESIDENT) == 0, "%s: unknown flags 0x%x", who, static_cast<unsigned>(flags));
  IRON_REQUIRE(q && k_new && v_new && k_cache && v_cache && angles && out && workspace, "%s: null pointer", who);
  IRON_REQUIRE(head_dim == kD, "%s: head_dim=%d (only 64 is supported)", who, head_dim);
  IRON_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "%s: n_heads=%d must be a multiple of n_kv_heads=%d", who, n_heads, n_kv_heads);
  const int G = n_heads / n_kv_heads;
  IRON_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "%s: group size %d not in {1,2,4,8}", who, G);
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
  a.ctr = static_cast<unsigned*>(workspace);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + decode_ctr_bytes(n_kv_heads));
  a.head_stride = decode_head_stride(G, max_len);
  a.pos_dev = pos_dev;
  a.pos = pos;
  a.max_len = max_len;
  a.angle_rows = angle_rows;
  a.nsplit = decode_nsplit(max_len);
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_kv_heads % kXcds == 0 && clear_counters)
    IRON_LAUNCH(gqa_clear_counters_kernel, dim3(1), dim3(kWave), 0, s, a.ctr, n_kv_heads);
  if (flags & IRON_GQA_KV_RESIDENT) {
    switch (G) {
      case 1: gqa_decode_dispatch<1, true>(a, n_kv_heads, s); break;
      case 2: gqa_decode_dispatch<2, true>(a, n_kv_heads, s); break;
      case 4: gqa_decode_dispatch<4, true>(a, n_kv_heads, s); break;
      default: gqa_decode_dispatch<8, true>(a, n_kv_heads, s); break;
    }
  } else {
    switch (G) {
      case 1: gqa_decode_dispatch<1, false>(a, n_kv_heads, s); break;
      case 2: gqa_decode_dispatch<2, false>(a, n_kv_heads, s); break;
      case 4: gqa_decode_dispatch<4, false>(a, n_kv_heads, s); break;
      default: gqa_decode_dispatch<8, false>(a, n_kv_heads, s); break;
    }
  }
  return check_launch(who);
}

extern "C" int iron_gqa_decode(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                               const float* angles, int angle_rows, void* out, void* workspace, int n_heads,
                               int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev, float scale,
                               void* stream) {
  return gqa_decode_launch("iron_gqa_decode", q, k_new, v_new, k_cache, v_cache, angles, angle_rows, out, workspace,
                           n_heads, n_kv_heads, head_dim, max_len, pos, pos_dev, scale, stream, false, 0);
}

extern "C" int iron_gqa_decode_ex(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                  const float* angles, int angle_rows, void* out, void* workspace, int n_heads,
                                  int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev, float scale,
                                  int flags, void* stream) {
  return gqa_decode_launch("iron_gqa_decode_ex", q, k_new, v_new, k_cache, v_cache, angles, angle_rows, out,
                           workspace, n_heads, n_kv_heads, head_dim, max_len, pos, pos_dev, scale, stream, false,
                           flags);
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
                           n_heads, n_kv_heads, head_dim, max_len, pos, pos_dev, scale, stream, true, 0);
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
  // K/V rows are addressed by 32-bit byte offsets from each head's base
  IRON_REQUIRE(kv_row_stride >= 0 && static_cast<long long>(seq_kv) * kv_row_stride * 2 < (1LL << 31) - 256,
               "iron_attention_prefill: seq_kv=%d x kv_row_stride=%lld spans more than 2 GiB", seq_kv, kv_row_stride);
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
