// Decode attention device code (split-K flash-decode), shared by the
// standalone entry points (attention.hip) and the one-launch decode step
// (decode_fused.hip).
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
// workgroup of the head to count itself in (an atomic in that L2) merges them,
// one wave per query head.
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
//
// The body (gqa_decode_chunk) takes its inputs and gives its output through an
// Io policy: PlainDecodeIo reads q / k_new / v_new from global memory written
// before the launch and stores the output there; the one-launch decode step
// supplies a policy that waits for them inside the launch.
#pragma once

#include "iron_common.hpp"
#include "trace.hpp"

#include <type_traits>

namespace iron {
namespace {

constexpr int kDecChunk = 64;  // cache positions per workgroup of 4 waves (16 per wave)
constexpr int kDecThreads = 256;
constexpr int kDecWaves1 = 8;  // waves per workgroup of the one-launch path on long caches (128 positions)
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
  void* trace;            // phase trace records (trace.hpp), or null
};

// One chunk's partial: G x 64 unnormalised outputs, then (maximum, sum) of
// each of the G heads as one 8-byte pair, padded to a whole number of
// 128-byte lines (head regions start on such a line too), so no two chunks'
// partials share a cache line: a line of them that a CU's L1 holds was
// written whole by one chunk on that CU.
template <int G>
constexpr int part_stride() {
  return (G * kD + 2 * G + 31) / 32 * 32;
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
    const float r = lower ? rot_sub(xo[e], c, xp[e], s) : rot_add(xo[e], c, xp[e], s);
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

// One decode step of KV head j for its G query heads; a workgroup of NW waves
// owns cache positions [CH s, CH s + CH), CH = 16 NW, wave w of it positions
// CH s + 16 w + [0, 16). NW = 4 (64 positions), or 8 (128 positions) for
// the one-launch path when that still gives at least one workgroup per CU:
// half the partials for the merge to read and half the workgroups to
// dispatch, for a longer wait on each CU's loads.
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
// active chunks to arrive returns the counter to zero and merges the head's
// partials from the L2 (gqa_merge_heads). No workgroup waits for another.
// Without MERGE the grid is (nsplit, Hkv) and gqa_combine_kernel merges.
// The cache rows one thread of the chunk at positions p0 + [0, 16 NW) of KV
// head j needs (they do not depend on the position: rows past it are masked
// or replaced later). K: lane l of wave w holds row p0 + 16 w + l % 16, dims 8 (l / 16) + [0, 8) (k0)
// and 32 + the same (k1). V: lane l of load u holds row 16 w + 8 u + l / 8,
// 16-byte chunk dec_v_slot(row, l % 8), which the body stores into slot l % 8
// of the wave's LDS block. Rows are clamped to the cache. RES: the caches stay
// resident between calls (a decode loop over all layers; ~134 MB at 4096
// positions fits the Infinity Cache while the weights stream past it), so
// the loads are ordinary, allocating loads (decode +0.9%); otherwise they are
// streaming loads, faster when the caches come from HBM every time.
struct DecodeKv {
  uint4 k0, k1, v0, v1;
};
template <bool RES>
__device__ __forceinline__ DecodeKv load_kv_rows(int tid, const uint16_t* k_cache, const uint16_t* v_cache,
                                                 int max_len, int p0, int j) {
  const int lane = tid & (kWave - 1), w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, cq = lane >> 4;
  const int wrow0 = p0 + 16 * w;
  const size_t hb = static_cast<size_t>(j) * max_len;
  auto ld_kv = [](const uint16_t* p) { return RES ? *reinterpret_cast<const uint4*>(p) : ld_stream16(p); };
  const int krow = min(wrow0 + r, max_len - 1);
  DecodeKv kv;
  kv.k0 = ld_kv(k_cache + (hb + krow) * kD + cq * 8);
  kv.k1 = ld_kv(k_cache + (hb + krow) * kD + (cq + 4) * 8);
  const int v0 = min(wrow0 + (lane >> 3), max_len - 1), v1 = min(wrow0 + 8 + (lane >> 3), max_len - 1);
  kv.v0 = ld_kv(v_cache + (hb + v0) * kD + dec_v_slot(lane >> 3, lane & 7) * 8);
  kv.v1 = ld_kv(v_cache + (hb + v1) * kD + dec_v_slot(8 + (lane >> 3), lane & 7) * 8);
  return kv;
}

// Inputs and output of one decode call in global memory (the standalone
// entry points): q, k_new and v_new were written before the launch, and the
// merged output goes to a.out.
template <int G>
struct PlainDecodeIo {
  static constexpr bool kEarly = true;
  static constexpr bool kStaleL1 = false;  // a launch's L1 starts invalidated (see gqa_decode_chunk's merge)
  static constexpr int kMergeChunks = 16;  // merge loads in flight per lane
  const DecodeArgs& a;
  __device__ __forceinline__ void new_kv(int j, int cq, uint4& kna, uint4& knb, uint4& vna, uint4& vnb) const {
    kna = *reinterpret_cast<const uint4*>(a.k_new + static_cast<size_t>(j) * kD + cq * 8);
    knb = *reinterpret_cast<const uint4*>(a.k_new + static_cast<size_t>(j) * kD + (cq + 4) * 8);
    vna = *reinterpret_cast<const uint4*>(a.v_new + static_cast<size_t>(j) * kD + cq * 8);
    vnb = *reinterpret_cast<const uint4*>(a.v_new + static_cast<size_t>(j) * kD + (cq + 4) * 8);
  }
  __device__ __forceinline__ void q_pair(int j, int t, uint16_t& qx, uint16_t& qp) const {
    const uint16_t* qh = a.q + static_cast<size_t>(j) * G * kD;
    qx = qh[t];
    qp = qh[t ^ 32];
  }
  __device__ __forceinline__ bool wait_inputs(int) const { return true; }
  __device__ __forceinline__ int thread() const { return threadIdx.x; }
  template <bool RES>
  __device__ __forceinline__ DecodeKv kv_rows(const DecodeArgs& d, int p0, int j) const {
    return load_kv_rows<RES>(threadIdx.x, d.k_cache, d.v_cache, d.max_len, p0, j);
  }
  __device__ __forceinline__ void store_out(size_t off, uint32_t lo, uint32_t hi) const {
    *reinterpret_cast<uint2*>(a.out + off) = make_uint2(lo, hi);
  }
};

template <int G, int NW, class Io>
__device__ void gqa_merge_heads(const DecodeArgs& a, int j, int nact, int tid, const Io& io);

// TR: the instance launched while a phase trace is armed (trace.hpp); the
// others carry no trace code.
template <int G, bool MERGE, bool RES, int NW, class Io, bool TR = false>
__device__ __forceinline__ void gqa_decode_chunk(const DecodeArgs& a, int s, int j, int pos, Io& io) {
  constexpr int D = kD;
  constexpr int NT = NW * kWave;   // threads
  constexpr int CH = NW * 16;      // cache positions
  constexpr int PS = part_stride<G>();
  __shared__ __attribute__((aligned(16))) uint16_t q_s[G * D];  // rotated q, bf16
  __shared__ float wm_s[NW][G], wl_s[NW][G];
  __shared__ __attribute__((aligned(16))) float wo_s[NW][G * D];
  __shared__ __attribute__((aligned(16))) unsigned char v_s[NW][16 * 128];  // each wave's 16 V rows

  const int tid = io.thread(), lane = tid & (kWave - 1), w = tid >> 6;
  // trace points: 0 start, 1 q in LDS, 2 scores and P V done, 3 partial stored
  // (acknowledged on the one-launch path), 4 counted in, 5 merged (last arriver)
  const unsigned twg = blockIdx.x + blockIdx.y * gridDim.x;
  void* const trace = TR ? a.trace : nullptr;
  unsigned long long t_start = 0;
  if constexpr (TR) t_start = trace_clock();
  if (pos < 0 || pos >= a.max_len || pos >= a.angle_rows) return;  // rejected on the host when pos is known
  const int L = pos + 1;
  const int p0 = s * CH;
  if (p0 >= L) return;
  const int r = lane & 15, cq = lane >> 4;
  const int wrow0 = p0 + 16 * w;
  const bool owner_wave = pos >= wrow0 && pos < wrow0 + 16;
  const bool owner = pos == wrow0 + r;  // the 4 lanes holding the new token's K row
  const size_t hb = static_cast<size_t>(j) * a.max_len;

  // Loads, oldest first: the new token's table entries and k/v (owner lanes),
  // then q and its table row, then the K rows, then the V rows. q is rotated
  // while K and V are still in flight (the waits below count only what the
  // rotation needs), and the scores wait for K alone. An Io whose q and new
  // k/v are produced during the same launch (Io::kEarly false) takes them
  // after the K/V loads are issued: its wait then overlaps them.
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
    if constexpr (Io::kEarly) io.new_kv(j, cq, kna, knb, vna, vnb);
  }
  constexpr int QN = (G * D + NT - 1) / NT;  // q elements per thread
  uint16_t qx[QN], qp[QN];
  float2 qa[QN];
#pragma unroll
  for (int e = 0; e < QN; ++e) {
    const int t = min(tid + NT * e, G * D - 1), i = (t % D) & 31;
    if constexpr (Io::kEarly) io.q_pair(j, t, qx[e], qp[e]);
    qa[e] = *reinterpret_cast<const float2*>(angrow + 2 * i);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the q loads ahead of the K/V loads
  // K rows (clamped: rows >= pos are replaced or masked below). RES: the caches
  // stay resident between calls (a decode loop over all layers; ~134 MB at 4096
  // positions fits the Infinity Cache while the weights stream past it), so the
  // K/V loads are ordinary, allocating loads (decode +0.9%). Otherwise they are
  // streaming loads, faster when the caches come from HBM every time.
  const DecodeKv kv = io.template kv_rows<RES>(a, p0, j);
  trace_write(trace, kTraceGqaDecode, twg, 0, t_start);
  uint4 k0 = kv.k0, k1 = kv.k1;
  unsigned char* vblk = v_s[w];
  const uint4 vraw[2] = {kv.v0, kv.v1};
  if constexpr (!Io::kEarly) {
    if (!io.wait_inputs(j)) return;  // workgroup-uniform
    if (owner) io.new_kv(j, cq, kna, knb, vna, vnb);
#pragma unroll
    for (int e = 0; e < QN; ++e) io.q_pair(j, min(tid + NT * e, G * D - 1), qx[e], qp[e]);
  }
#pragma unroll
  for (int e = 0; e < QN; ++e) {
    const int t = tid + NT * e;
    if (t < G * D) {
      const float x = bf16_to_f32(qx[e]), xp = bf16_to_f32(qp[e]);
      q_s[t] = f32_to_bf16((t % D) < 32 ? rot_sub(x, qa[e].x, xp, qa[e].y) : rot_add(x, qa[e].x, xp, qa[e].y));
    }
  }
  // barrier without a wait for the K/V loads in flight (__syncthreads would
  // wait for all of them); the memory clobber keeps the q_s accesses on their sides
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  trace_stamp(trace, kTraceGqaDecode, twg, 1);
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
  trace_stamp(trace, kTraceGqaDecode, twg, 2);

  // the chunk's partial: the four waves merged
  float* part = a.part + static_cast<size_t>(j) * a.head_stride + static_cast<size_t>(s) * PS;
  for (int t = tid; t < G * D; t += NT) {
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
    if (t % D == 0) *reinterpret_cast<float2*>(part + G * D + 2 * g) = make_float2(M, l);
  }
  if constexpr (!MERGE) trace_stamp(trace, kTraceGqaDecode, twg, 3);
  if constexpr (MERGE) {
    __shared__ int last_s;
    const int nact = (L + CH - 1) / CH;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores have reached the L2
    __syncthreads();
    trace_stamp(trace, kTraceGqaDecode, twg, 3);
    if (tid == 0) {  // an atomic in the XCD's L2, where the partials are
      unsigned* c = a.ctr + static_cast<size_t>(j) * kCtrStride;
      const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      const int last = old == static_cast<unsigned>(nact - 1);
      if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      last_s = last;
    }
    __syncthreads();
    trace_stamp(trace, kTraceGqaDecode, twg, 4);
    if (!last_s) return;
    // An Io whose persistent workgroups merge again later (Io::kStaleL1) may
    // hold lines of an earlier merge's partials in this CU's L1: an
    // agent-scope invalidate first (~0.9 us, so not for a fresh launch, where
    // the L1 starts invalidated and holds at most lines a chunk on this CU
    // wrote whole: part_stride).
    if constexpr (Io::kStaleL1) asm volatile("buffer_inv sc1" ::: "memory");
    gqa_merge_heads<G, NW>(a, j, nact, tid, io);
    trace_stamp(trace, kTraceGqaDecode, twg, 5);
  }
}

// The merge of KV head j's nact chunk partials by the workgroup that finished
// last, one wave per query head (heads w, w + NW, ...; waves >= G idle).
// Lane -> output quad qd = lane % 16 (dims 4 qd .. 4 qd + 3) and chunk slice
// r = lane / 16 (chunks r, r + 4, ...): per chunk one 16-byte load of the
// outputs and one 8-byte load of (maximum, sum), a round of B chunks per lane
// all in flight together (B = 8 or 16 by the active count, capped by
// Io::kMergeChunks; more chunks take more rounds). Each slice folds its chunks
// with a running maximum and the four slices meet by permlane swaps: no LDS
// and no barrier. The partials were written to the XCD's L2 by other CUs
// and are read with plain loads (see the caller on this CU's L1).
// Every sum runs in a fixed order: the result depends only on the data.
template <int G, int NW, class Io>
__device__ void gqa_merge_heads(const DecodeArgs& a, int j, int nact, int tid, const Io& io) {
  constexpr int D = kD;
  constexpr int PS = part_stride<G>();
  constexpr int NS = kWave / (D / 4);  // chunk slices per wave
  const int lane = tid & (kWave - 1), w = tid >> 6, qd = lane & (D / 4 - 1), r = lane / (D / 4);
  const float* base = a.part + static_cast<size_t>(j) * a.head_stride;
  const int span = (nact + NS - 1) / NS;  // chunks of slice 0
  for (int g = w; g < G; g += NW) {
    float m = -INFINITY, l = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto round = [&](auto b_tag, int c0) {
      constexpr int B = decltype(b_tag)::value;
      float2 st[B];
      float4 ob[B];
#pragma unroll
      for (int b = 0; b < B; ++b) {  // chunk c0 + r + NS b (past nact: chunk nact - 1, dropped below)
        const float* pk = base + static_cast<size_t>(min(c0 + r + NS * b, nact - 1)) * PS;
        st[b] = *reinterpret_cast<const float2*>(pk + G * D + 2 * g);
        ob[b] = *reinterpret_cast<const float4*>(pk + g * D + 4 * qd);
      }
      float bm = m;
#pragma unroll
      for (int b = 0; b < B; ++b)
        if (c0 + r + NS * b < nact) bm = fmaxf(bm, st[b].x);  // a live chunk's maximum is finite
      if (bm == -INFINITY) return;                            // no live chunk in this slice
      const float keep = exp2_weight(m - bm);                 // 0 while m is -inf
      acc.x *= keep;
      acc.y *= keep;
      acc.z *= keep;
      acc.w *= keep;
      l *= keep;
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const float wgt = c0 + r + NS * b < nact ? exp2_weight(st[b].x - bm) : 0.f;
        acc.x = fmaf(wgt, ob[b].x, acc.x);
        acc.y = fmaf(wgt, ob[b].y, acc.y);
        acc.z = fmaf(wgt, ob[b].z, acc.z);
        acc.w = fmaf(wgt, ob[b].w, acc.w);
        l = fmaf(wgt, st[b].y, l);
      }
      m = bm;
    };
    constexpr int BMAX = Io::kMergeChunks;
    if (span <= 4)
      round(std::integral_constant<int, 4>{}, 0);
    else if (span <= 8 || BMAX < 16)
      for (int c0 = 0; c0 < nact; c0 += NS * 8) round(std::integral_constant<int, 8>{}, c0);
    else
      for (int c0 = 0; c0 < nact; c0 += NS * BMAX) round(std::integral_constant<int, BMAX>{}, c0);
    // the four slices: rows r and r ^ 2, then r and r ^ 1 (x: the lower row)
    auto fold = [&](auto split) {
      float mx, my;
      split(m, mx, my);
      const float mn = fmaxf(mx, my);  // finite: slice 0 holds chunk 0
      const float fx = mx == -INFINITY ? 0.f : exp2_weight(mx - mn), fy = my == -INFINITY ? 0.f : exp2_weight(my - mn);
      auto mix = [&](float& v) {
        float x, y;
        split(v, x, y);
        v = fmaf(fx, x, fy * y);
      };
      mix(acc.x);
      mix(acc.y);
      mix(acc.z);
      mix(acc.w);
      mix(l);
      m = mn;
    };
    fold([](float v, float& x, float& y) { split32(v, x, y); });
    fold([](float v, float& x, float& y) { split16(v, x, y); });
    if (r == 0) {
      const float rl = __builtin_amdgcn_rcpf(l);
      io.store_out(static_cast<size_t>(j * G + g) * D + 4 * qd, cvt_pk_bf16(acc.x * rl, acc.y * rl),
                   cvt_pk_bf16(acc.z * rl, acc.w * rl));
    }
  }
}

// The arguments that the position load and the first K/V, q and table loads
// need come first, as copies of their DecodeArgs fields: the dispatch preloads
// them into SGPRs (the kernarg preload count of the including file's build),
// so a workgroup issues the position load without waiting for an argument
// fetch, and the fetch of the other fields overlaps it.
template <int G, bool MERGE, bool RES, int NW, bool TR>
__global__ __launch_bounds__(NW * kWave) void gqa_decode_kernel(const int* pos_dev, const uint16_t* k_cache,
                                                                const uint16_t* v_cache, const float* angles,
                                                                const uint16_t* q, int pos, int nsplit, int max_len,
                                                                int angle_rows, DecodeArgs a) {
  int s, j;
  if constexpr (MERGE) {
    const int n = blockIdx.x, t = n / kXcds;
    j = n % kXcds + kXcds * (t / nsplit);
    s = t % nsplit;
  } else {
    s = blockIdx.x;
    j = blockIdx.y;
  }
  DecodeArgs b = a;
  b.k_cache = const_cast<uint16_t*>(k_cache);
  b.v_cache = const_cast<uint16_t*>(v_cache);
  b.angles = angles;
  b.q = q;
  b.nsplit = nsplit;
  b.max_len = max_len;
  b.angle_rows = angle_rows;
  const int p = pos_dev ? *pos_dev : pos;
  // k_new and v_new are fetched here, together with the position: fetched where
  // the chunk first uses them (after the position checks), they added a
  // second argument round trip ahead of the K/V loads
  asm volatile("" ::"s"(b.k_new), "s"(b.v_new));
  PlainDecodeIo<G> io{b};
  gqa_decode_chunk<G, MERGE, RES, NW, PlainDecodeIo<G>, TR>(b, s, j, p, io);
}

// Launch of gqa_decode_kernel with its leading copies taken from `a`.
#define IRON_GQA_DECODE_LAUNCH(KERNEL, GRID, BLOCK, STREAM, A)                                                  \
  IRON_LAUNCH(KERNEL, GRID, BLOCK, 0, STREAM, (A).pos_dev, static_cast<const uint16_t*>((A).k_cache),          \
              static_cast<const uint16_t*>((A).v_cache), (A).angles, (A).q, (A).pos, (A).nsplit, (A).max_len,     \
              (A).angle_rows, A)

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
    mb[b] = pk[G * D + 2 * g];
    lb[b] = pk[G * D + 2 * g + 1];
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
        mb[b] = pk[G * D + 2 * g];
        lb[b] = pk[G * D + 2 * g + 1];
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

}  // namespace
}  // namespace iron
