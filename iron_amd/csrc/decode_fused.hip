// One decode step of a Llama-3.2-1B-shaped model (hidden 2048, 32/8 GQA
// heads of 64, FFN 8192, int4-group-32 linears) in a single launch: the token
// selection and every layer's qkv GEMV, attention, o_proj, SwiGLU pair and
// down projection. Only the LM head (iron_llama_decode_head) follows it.
//
// Dataflow instead of launch boundaries. The grid lists the work in
// dependency order (select; then per layer qkv rows, attention chunks, o rows,
// gate/up rows, down rows); a workgroup only ever waits for workgroups with
// lower ids. Workgroups are dispatched in id order, so the lowest unfinished
// workgroup always has every input it waits for: the launch always drains.
// Each GEMV workgroup issues its weight loads first (they do not depend on the
// step) and only then waits for its input vector, so the weights of the next
// stage stream while the current one finishes; each attention workgroup
// issues its K/V cache loads before it waits for q/k/v.
//
// Exchange. Producers publish their outputs into an exchange area as 8-byte
// pairs (32 data bits, 32 tag bits) with agent-scope stores (sc1: written
// through to where every XCD's loads see them); consumers read them with
// agent-scope loads and accept a pair only when its tag is the step's epoch.
// 8-byte halves of a 16-byte access are single-copy atomic, so a pair never
// mixes data of two steps; no counter, fence or atomic read-modify-write is
// involved. The epoch is read by every workgroup at its start and advanced by
// the head GEMV after the launch (iron_llama_decode_head), so a step's tags
// never match what an earlier step left. A consumer first polls one pair per
// XCD (the one written by that XCD's last producer workgroup), then loads the
// whole vector once and re-polls only pairs that are not there yet.
//
// Bounded waits. Every wait gives up after `wait_us` (s_memrealtime, 100 MHz)
// or as soon as the status word is non-zero; the workgroup then records its
// stage bit in the status word and returns, and every later wait sees the
// status and returns too, so a failed step ends in bounded time with the
// cause in the status word. The caller reads the status word after the step.
//
// Arithmetic. Each role computes exactly what the separate kernels compute
// (the same int4 group products, DPP reductions, norm scale, SiLU and residual
// order, and the shared decode attention body), so the step's logits are
// bit-identical to the 82-launch step.
#include "iron_common.hpp"
#include "i4_dot.hpp"
#include "decode_attn.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

constexpr int kE = 2048;                         // hidden size
constexpr int kF = 8192;                         // FFN size
constexpr int kNH = 32, kNKV = 8, kGQ = 4;       // query heads, KV heads, heads per KV head
constexpr int kQKV = (kNH + 2 * kNKV) * kD;      // 3072 q|k|v rows

// Workgroups per stage (256 threads each)
constexpr int kWgSel = 8;         // the select workgroup, padded to one per XCD
constexpr int kWgQkv = kQKV / 4;  // one row per wave
constexpr int kWgO = kE / 4;      // one row per wave
constexpr int kWgPair = kF / 8;   // two gate and two up rows per wave
constexpr int kWgDown = kE / 8;   // two rows (K = 8192) per wave

// Exchange area in 8-byte pairs: the position pair, then per layer its input
// x, qkv, attention output, x after o_proj, h; the last layer's output x
// follows the last layer.
constexpr int kPosPairs = 16;
constexpr int kOffQkv = kE / 2;
constexpr int kOffAtt = kOffQkv + kQKV / 2;
constexpr int kOffX1 = kOffAtt + kNH * kD / 2;
constexpr int kOffH = kOffX1 + kE / 2;
constexpr int kLayerPairs = kOffH + kF / 2;  // 8704
__host__ __device__ constexpr int layer_pairs(int l) { return kPosPairs + l * kLayerPairs; }

// The GEMVs' norm modes used here (gemv.hip): none, or the outputs scaled by
// rsqrt(mean(x^2) + eps) with the norm weight folded into the matrix.
enum : int { NORM_NONE = 0, NORM_SCALE = 2 };

// Status bits: which wait gave up.
enum : unsigned {
  kStX = 1u,     // qkv: layer input
  kStPos = 2u,   // attention: position
  kStQkv = 4u,   // attention: q, k, v
  kStAtt = 8u,   // o_proj: attention output
  kStX1 = 16u,   // gate/up: x after o_proj
  kStH = 32u,    // down: h
  kStRes = 64u,  // a residual
};

struct FusedArgs {
  const IronDecodeLayer* layers;  // device table, n_layers entries
  int n_layers;
  int nsplit;  // attention chunks per KV head
  int max_len;
  int angle_rows;
  const unsigned long long* keys;  // argmax keys of the previous head GEMV
  int n_keys;
  const uint16_t* embed;
  int vocab;
  int* token;
  int* pos;
  int* history;
  int history_cap;
  const float* angles;
  float* part;  // attention partials
  unsigned* ctr;  // attention arrival counters (kept at zero between calls)
  long long head_stride;
  float scale_log2;
  float eps;
  unsigned char* xch;  // exchange area
  uint16_t* x_out;     // plain copy of the last layer's output (the head's input)
  const unsigned* epoch;
  unsigned* status;
  unsigned wait_ticks;  // 100 MHz ticks
};

typedef unsigned u32x4_v __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_v __attribute__((ext_vector_type(2)));
constexpr int kSc1 = 16;  // cache-policy bits of the buffer builtins: sc1 (agent scope)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t xch_rsrc(const unsigned char* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(base), 0, 0x7fffffff, kBufferFlags);
}
// pairs p and p + 1 (p even)
__device__ __forceinline__ u32x4_v ld_pairs2(__amdgpu_buffer_rsrc_t r, int p) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, p * 8, 0, kSc1);
}
__device__ __forceinline__ u32x2_v ld_pair(__amdgpu_buffer_rsrc_t r, int p) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, p * 8, 0, kSc1);
}
__device__ __forceinline__ void st_pairs2(__amdgpu_buffer_rsrc_t r, int p, uint32_t d0, uint32_t d1, unsigned tag) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4_v{d0, tag, d1, tag}, r, p * 8, 0, kSc1);
}
__device__ __forceinline__ void st_pair(__amdgpu_buffer_rsrc_t r, int p, uint32_t d, unsigned tag) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_v{d, tag}, r, p * 8, 0, kSc1);
}

__device__ __forceinline__ unsigned long long now_ticks() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ unsigned read_status(const unsigned* status) {
  return __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void give_up(unsigned* status, unsigned bit) {
  __hip_atomic_fetch_or(status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Workgroup barrier for LDS only: the weight and cache loads in flight are not waited for.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// XCD-contiguous tile of local workgroup b of a stage of nb workgroups (stage
// starts are multiples of 8, so b % 8 is the XCD): each XCD owns one
// contiguous run of tiles.
__device__ __forceinline__ int stage_tile(int b, int nb) { return (b & 7) * (nb >> 3) + (b >> 3); }
// The last pair written by the last workgroup on XCD x of a GEMV stage (pw pairs per workgroup).
__device__ __forceinline__ int gemv_sentinel(int x, int nb, int pw) { return (x * (nb >> 3) + (nb >> 3) - 1) * pw + pw - 1; }

// Waits until pairs [p0, p0 + NP) carry `tag` and leaves their data words in
// dst[0, NP) (LDS). Lanes 0-7 of wave 0 first poll sent[x] (relative to p0),
// lane 8 the status word; then every thread loads its share once and re-polls
// only pairs still missing. Whole workgroup (flag: two LDS words); false,
// for every thread alike, when it gave up.
template <int NP>
__device__ bool wait_vector(__amdgpu_buffer_rsrc_t r, unsigned* status, int p0, const int* sent, unsigned tag,
                            unsigned limit, unsigned bit, uint32_t* dst, int* flag) {
  static_assert(NP % 512 == 0, "two pairs per 16-byte load, 256 threads");
  const int tid = threadIdx.x;
  if (tid < kWave) {
    const unsigned long long t0 = now_ticks();
    int fail = 0;
    for (;;) {
      const u32x2_v v = ld_pair(r, p0 + sent[tid & 7]);
      const unsigned st = tid == 8 ? read_status(status) : 0u;
      if (__builtin_amdgcn_ballot_w64(st != 0u)) {
        fail = 1;
        break;
      }
      if (!__builtin_amdgcn_ballot_w64(tid < 8 && v[1] != tag)) break;
      if (now_ticks() - t0 > limit) {
        fail = 2;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (tid == 0) {
      flag[0] = fail;
      flag[1] = 0;
    }
  }
  lds_barrier();
  const int f = flag[0];
  if (f) {
    if (f == 2 && tid == 0) give_up(status, bit);
    return false;
  }
  constexpr int NL = NP / 512;
  u32x4_v v[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) v[i] = ld_pairs2(r, p0 + 2 * (tid + 256 * i));
  bool ok = true;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    if (v[i][1] != tag || v[i][3] != tag) {  // rare: re-poll this pair of pairs
      const unsigned long long t0 = now_ticks();
      while (ok && (v[i][1] != tag || v[i][3] != tag)) {
        if (read_status(status) != 0u || now_ticks() - t0 > limit) ok = false;
        __builtin_amdgcn_s_sleep(1);
        v[i] = ld_pairs2(r, p0 + 2 * (tid + 256 * i));
      }
    }
    *reinterpret_cast<uint2*>(dst + 2 * (tid + 256 * i)) = make_uint2(v[i][0], v[i][2]);
  }
  if (!ok) {
    give_up(status, bit);
    flag[1] = 1;
  }
  lds_barrier();
  return flag[1] == 0;
}

// The data word of pair p (a residual: rows 2p, 2p + 1), polled by the whole
// wave. The pair is complete by the time a stage needs it (the stage's input
// depends on it), so the wait is a guard: if it gives up, the status records
// it and the caller goes on with whatever it read (the step has failed; every
// wave still reaches the workgroup's barriers).
__device__ __forceinline__ uint32_t wait_pair(__amdgpu_buffer_rsrc_t r, unsigned* status, int p, unsigned tag,
                                              unsigned limit) {
  u32x2_v v = ld_pair(r, p);
  if (v[1] != tag) {
    const unsigned long long t0 = now_ticks();
    while (v[1] != tag) {
      const unsigned s = read_status(status);
      if (s != 0u || now_ticks() - t0 > limit) {
        if (s == 0u) give_up(status, kStRes);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      v = ld_pair(r, p);
    }
  }
  return v[0];
}

// A GEMV stage's workgroup: rows (tile * 4 + wave) * R + [0, R) of an int4
// group-32 matrix (K = 2048 * GPL), the arithmetic of gemv_i4_fast<GPL, R, 1,
// PAIR, NM> (signed codes, no epilogue). Input: the KP-pair vector at in_p0;
// residual: the pairs at res_p0; output: pairs at out_p0 (+ plain bf16 copy).
template <int GPL, int R, bool PAIR, int NM, bool RESID>
__device__ void gemv_role(const FusedArgs& a, int tile, const uint8_t* codes, const uint16_t* scales,
                          const uint8_t* codes2, const uint16_t* scales2, int in_p0, const int* sent, unsigned in_bit,
                          int res_p0, int out_p0, uint16_t* plain, unsigned tag, uint32_t* xs, int* flag) {
  constexpr int G = GPL * kWave;   // groups per row
  constexpr int K = G * 32;
  constexpr int KP = K / 2;        // input pairs
  constexpr size_t crow = static_cast<size_t>(G) * 16;
  constexpr uint32_t kMagic = 0x43084308u;  // signed codes
  constexpr float kOffset = 136.f;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int row0 = (tile * 4 + wave) * R;
  const int g0 = lane;

  // The weights first: nothing of this step is needed to fetch them.
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
  __builtin_amdgcn_sched_barrier(0);

  const __amdgpu_buffer_rsrc_t xr_ = xch_rsrc(a.xch);
  if (!wait_vector<KP>(xr_, a.status, in_p0, sent, tag, a.wait_ticks, in_bit, xs, flag)) return;
  float rres[R];
  if (RESID) {
    const uint32_t d = wait_pair(xr_, a.status, res_p0 + (row0 >> 1), tag, a.wait_ticks);
    if (R == 2) {
      rres[0] = lo_bf16(d);
      if (R > 1) rres[R - 1] = hi_bf16(d);
    } else {
      rres[0] = (row0 & 1) ? hi_bf16(d) : lo_bf16(d);
    }
  }

  uint4 xrv[GPL][4];
  const uint4* xv = reinterpret_cast<const uint4*>(xs);
#pragma unroll
  for (int j = 0; j < GPL; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) xrv[j][q] = xv[(g0 + j * kWave) * 4 + q];
  float inv = 1.f;
  if (NM == NORM_SCALE) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < GPL; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) ss = sumsq_chunk(xrv[j][q], ss);
    ss = wave_sum(ss);
    inv = inv_rms(ss, K, a.eps);
  }
  XGroup xg[GPL];
#pragma unroll
  for (int j = 0; j < GPL; ++j) build_xgroup(xrv[j], xg[j]);
  uint16_t outv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.f, acc2 = 0.f;
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
      const float d = i4_group_total(cw[r][j], xg[j], kMagic, kOffset);
      acc = fmaf(bf16_to_f32(sc[r][j]), d, acc);
      if (PAIR) {
        const float d2 = i4_group_total(cw2[r][j], xg[j], kMagic, kOffset);
        acc2 = fmaf(bf16_to_f32(sc2[r][j]), d2, acc2);
      }
    }
    float t = wave_sum(acc);
    float t2 = PAIR ? wave_sum(acc2) : 0.f;
    if (NM == NORM_SCALE) {
      t *= inv;
      t2 *= inv;
    }
    float v = PAIR ? silu_f32(t) * t2 : t;
    if (RESID) v += rres[r];
    outv[r] = f32_to_bf16(v);
  }
  if (R == 2) {
    if (lane == 0) {
      const uint32_t d = static_cast<uint32_t>(outv[0]) | (static_cast<uint32_t>(outv[R - 1]) << 16);
      st_pair(xr_, out_p0 + (row0 >> 1), d, tag);
      if (plain) *reinterpret_cast<uint32_t*>(plain + row0) = d;
    }
  } else {  // four rows of the workgroup: one 16-byte store
    __shared__ uint16_t rows_s[4];
    if (lane == 0) rows_s[wave] = outv[0];
    lds_barrier();
    if (tid == 0) {
      const uint32_t d0 = rows_s[0] | (static_cast<uint32_t>(rows_s[1]) << 16);
      const uint32_t d1 = rows_s[2] | (static_cast<uint32_t>(rows_s[3]) << 16);
      st_pairs2(xr_, out_p0 + tile * 2, d0, d1, tag);
      if (plain) *reinterpret_cast<uint2*>(plain + tile * 4) = make_uint2(d0, d1);
    }
  }
}

// The attention's Io inside the step: q (4 heads), k_new and v_new of KV head j
// are waited for in the exchange area and staged in LDS (st[0..255] q,
// [256..319] k, [320..383] v as bf16); the merged output is published as pairs.
struct FusedDecodeIo {
  static constexpr bool kEarly = false;
  const FusedArgs& fa;
  int qkv_p0, att_p0;
  unsigned tag;
  uint32_t* st;  // 192 words of LDS
  int* flag;
  __device__ __forceinline__ bool wait_inputs(int j) const {
    const __amdgpu_buffer_rsrc_t r = xch_rsrc(fa.xch);
    const int tid = threadIdx.x;
    if (tid == 0) flag[2] = 0;
    lds_barrier();
    if (tid < 96) {  // 192 pairs, two per thread: q (64 loads), k (16), v (16)
      const int p = tid < 64 ? j * (kGQ * kD / 2) + 2 * tid
                             : (tid < 80 ? kNH * kD / 2 + j * (kD / 2) + 2 * (tid - 64)
                                         : (kNH + kNKV) * kD / 2 + j * (kD / 2) + 2 * (tid - 80));
      u32x4_v v = ld_pairs2(r, qkv_p0 + p);
      if (v[1] != tag || v[3] != tag) {
        const unsigned long long t0 = now_ticks();
        while (v[1] != tag || v[3] != tag) {
          const unsigned s = read_status(fa.status);
          if (s != 0u || now_ticks() - t0 > fa.wait_ticks) {
            if (s == 0u) give_up(fa.status, kStQkv);
            flag[2] = 1;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          v = ld_pairs2(r, qkv_p0 + p);
        }
      }
      *reinterpret_cast<uint2*>(st + 2 * tid) = make_uint2(v[0], v[2]);
    }
    lds_barrier();
    return flag[2] == 0;
  }
  __device__ __forceinline__ void q_pair(int, int t, uint16_t& qx, uint16_t& qp) const {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(st);
    qx = q[t];
    qp = q[t ^ 32];
  }
  __device__ __forceinline__ void new_kv(int, int cq, uint4& kna, uint4& knb, uint4& vna, uint4& vnb) const {
    const uint4* kv = reinterpret_cast<const uint4*>(st + kGQ * kD / 2);  // k at 16-byte chunk 0.., v at 8..
    kna = kv[cq];
    knb = kv[cq + 4];
    vna = kv[8 + cq];
    vnb = kv[8 + cq + 4];
  }
  template <bool RES>
  __device__ __forceinline__ DecodeKv kv_rows(const DecodeArgs& d, int s, int j) const {
    return load_kv_rows<RES>(d.k_cache, d.v_cache, d.max_len, s, j);
  }
  __device__ __forceinline__ void store_out(size_t off, uint32_t lo, uint32_t hi) const {
    st_pairs2(xch_rsrc(fa.xch), att_p0 + static_cast<int>(off >> 1), lo, hi, tag);
  }
};

template <bool RES>
__device__ void attention_role(const FusedArgs& a, const IronDecodeLayer& L, int n, int lbase, unsigned tag,
                               uint32_t* st, int* flag) {
  const int j = n % kXcds, s = n / kXcds;  // all chunks of KV head j on one XCD
  const __amdgpu_buffer_rsrc_t r = xch_rsrc(a.xch);
  // the position (published by the select workgroup at the start of the step),
  // polled by wave 0 and shared through LDS so that every wave takes the same path
  if (threadIdx.x < kWave) {
    u32x2_v pv = ld_pair(r, 0);
    int got = 1;
    if (pv[1] != tag) {
      const unsigned long long t0 = now_ticks();
      while (pv[1] != tag) {
        const unsigned sv = read_status(a.status);
        if (sv != 0u || now_ticks() - t0 > a.wait_ticks) {
          if (sv == 0u && threadIdx.x == 0) give_up(a.status, kStPos);
          got = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        pv = ld_pair(r, 0);
      }
    }
    if (threadIdx.x == 0) {
      flag[0] = got;
      flag[1] = static_cast<int>(pv[0]);
    }
  }
  lds_barrier();
  if (!flag[0]) return;
  const int pos = flag[1];
  if (pos < 0 || pos >= a.max_len || pos >= a.angle_rows) {
    // never for a position the host accepted; publish zeros so the step drains
    if (s == 0 && threadIdx.x < kGQ * kD / 4)
      st_pairs2(r, lbase + kOffAtt + j * (kGQ * kD / 2) + 2 * threadIdx.x, 0u, 0u, tag);
    return;
  }
  DecodeArgs d;
  d.q = d.k_new = d.v_new = nullptr;
  d.k_cache = static_cast<uint16_t*>(L.k_cache);
  d.v_cache = static_cast<uint16_t*>(L.v_cache);
  d.angles = a.angles;
  d.out = nullptr;
  d.part = a.part;
  d.ctr = a.ctr;
  d.head_stride = a.head_stride;
  d.pos_dev = nullptr;
  d.pos = pos;
  d.max_len = a.max_len;
  d.angle_rows = a.angle_rows;
  d.nsplit = a.nsplit;
  d.scale_log2 = a.scale_log2;
  FusedDecodeIo io{a, lbase + kOffQkv, lbase + kOffAtt, tag, st, flag};
  gqa_decode_chunk<kGQ, true, RES>(d, s, j, pos, io);
}

// Token selection (the previous head's argmax keys), bookkeeping, and the
// embedding row as layer 0's input: select_embed_kernel's work by 256 threads,
// with the position and x published to the exchange area.
__device__ void select_role(const FusedArgs& a, unsigned tag) {
  __shared__ unsigned long long ks[4];
  __shared__ int tok_s;
  const int p = *a.pos;
  constexpr int U = 32;
  unsigned long long best = 0;
  for (int base = 0; base < a.n_keys; base += 256 * U) {
    unsigned long long k[U];
#pragma unroll
    for (int u = 0; u < U; ++u) k[u] = a.keys[min(base + u * 256 + static_cast<int>(threadIdx.x), a.n_keys - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u) best = k[u] > best ? k[u] : best;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off, kWave);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) ks[threadIdx.x >> 6] = best;
  __syncthreads();
  const __amdgpu_buffer_rsrc_t r = xch_rsrc(a.xch);
  if (threadIdx.x == 0) {
    unsigned long long b = ks[0];
    for (int w = 1; w < 4; ++w) b = ks[w] > b ? ks[w] : b;
    int tok = static_cast<int>(argmax_key_index(b));
    if (tok < 0 || tok >= a.vocab) tok = 0;
    tok_s = tok;
    a.token[0] = tok;
    if (a.history && p >= 0 && p < a.history_cap) a.history[p] = tok;
    *a.pos = p + 1;
    st_pair(r, 0, static_cast<uint32_t>(p + 1), tag);
  }
  __syncthreads();
  const uint4 v = reinterpret_cast<const uint4*>(a.embed + static_cast<size_t>(tok_s) * kE)[threadIdx.x];
  st_pairs2(r, layer_pairs(0) + 4 * threadIdx.x, v.x, v.y, tag);
  st_pairs2(r, layer_pairs(0) + 4 * threadIdx.x + 2, v.z, v.w, tag);
}

// RES: the attention's K/V loads are allocating loads (IRON_GQA_KV_RESIDENT).
template <bool RES>
__global__ __launch_bounds__(256) void decode_step_kernel(FusedArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t xs[kF / 2];  // a stage's input vector
  __shared__ int flag[4];
  const unsigned tag = *a.epoch;
  const int b = blockIdx.x;
  if (b < kWgSel) {
    if (b == 0) select_role(a, tag);
    return;
  }
  const int per = kWgQkv + kNKV * a.nsplit + kWgO + kWgPair + kWgDown;
  const int l = (b - kWgSel) / per;
  int r = (b - kWgSel) % per;
  const IronDecodeLayer L = a.layers[l];
  const int base = layer_pairs(l);
  int sent[8];
  if (r < kWgQkv) {  // qkv = Wqkv' x * rms(x); input from the select (layer 0) or the previous down
#pragma unroll
    for (int x = 0; x < 8; ++x) sent[x] = l == 0 ? kE / 2 - 1 : gemv_sentinel(x, kWgDown, 4);
    gemv_role<1, 1, false, NORM_SCALE, false>(a, stage_tile(r, kWgQkv), static_cast<const uint8_t*>(L.qkv_codes),
                                              static_cast<const uint16_t*>(L.qkv_scales), nullptr, nullptr, base,
                                              sent, kStX, 0, base + kOffQkv, nullptr, tag, xs, flag);
    return;
  }
  r -= kWgQkv;
  if (r < kNKV * a.nsplit) {
    attention_role<RES>(a, L, r, base, tag, xs, flag);
    return;
  }
  r -= kNKV * a.nsplit;
  if (r < kWgO) {  // x1 = x + Wo attn
#pragma unroll
    for (int x = 0; x < 8; ++x) sent[x] = x * (kGQ * kD / 2) + kGQ * kD / 2 - 1;
    gemv_role<1, 1, false, NORM_NONE, true>(a, stage_tile(r, kWgO), static_cast<const uint8_t*>(L.o_codes),
                                            static_cast<const uint16_t*>(L.o_scales), nullptr, nullptr,
                                            base + kOffAtt, sent, kStAtt, base, base + kOffX1, nullptr, tag, xs,
                                            flag);
    return;
  }
  r -= kWgO;
  if (r < kWgPair) {  // h = silu(Wg' x1 * rms) * (Wu' x1 * rms)
#pragma unroll
    for (int x = 0; x < 8; ++x) sent[x] = gemv_sentinel(x, kWgO, 2);
    gemv_role<1, 2, true, NORM_SCALE, false>(a, stage_tile(r, kWgPair), static_cast<const uint8_t*>(L.gate_codes),
                                             static_cast<const uint16_t*>(L.gate_scales),
                                             static_cast<const uint8_t*>(L.up_codes),
                                             static_cast<const uint16_t*>(L.up_scales), base + kOffX1, sent, kStX1, 0,
                                             base + kOffH, nullptr, tag, xs, flag);
    return;
  }
  r -= kWgPair;
  // x' = x1 + Wd h (the next layer's input; the last layer also writes x_out)
#pragma unroll
  for (int x = 0; x < 8; ++x) sent[x] = gemv_sentinel(x, kWgPair, 4);
  gemv_role<4, 2, false, NORM_NONE, true>(a, stage_tile(r, kWgDown), static_cast<const uint8_t*>(L.down_codes),
                                          static_cast<const uint16_t*>(L.down_scales), nullptr, nullptr, base + kOffH,
                                          sent, kStH, base + kOffX1, layer_pairs(l + 1),
                                          l == a.n_layers - 1 ? a.x_out : nullptr, tag, xs, flag);
}

}  // namespace
}  // namespace iron

using namespace iron;

extern "C" long long iron_llama_decode_fused_exchange_bytes(int n_layers) {
  if (n_layers <= 0 || n_layers > 1024) return -1;
  return static_cast<long long>(layer_pairs(n_layers) + kE / 2) * 8;
}

extern "C" int iron_llama_decode_fused(const IronDecodeLayer* layers, int n_layers, const void* keys, int n_keys,
                                       const void* embed, int vocab, int* token, int* pos, int* history,
                                       int history_cap, const float* angles, int angle_rows, int max_len, float scale,
                                       float eps, void* attn_workspace, void* exchange, void* x_out,
                                       const unsigned* epoch, unsigned* status, unsigned wait_us, int flags,
                                       void* stream) {
  const char* who = "iron_llama_decode_fused";
  IRON_REQUIRE((flags & ~IRON_GQA_KV_RESIDENT) == 0, "%s: unknown flags 0x%x", who, static_cast<unsigned>(flags));
  IRON_REQUIRE(layers && keys && embed && token && pos && angles && attn_workspace && exchange && x_out && epoch &&
                   status,
               "%s: null pointer", who);
  IRON_REQUIRE(n_layers > 0 && n_layers <= 1024, "%s: n_layers=%d", who, n_layers);
  IRON_REQUIRE(n_keys > 0 && vocab > 0, "%s: n_keys=%d vocab=%d", who, n_keys, vocab);
  IRON_REQUIRE(max_len > 0 && max_len % kDecChunk == 0 && angle_rows > 0,
               "%s: max_len=%d must be a positive multiple of %d", who, max_len, kDecChunk);
  IRON_REQUIRE(wait_us >= 1 && wait_us <= 10000000u, "%s: wait_us=%u outside [1, 1e7]", who, wait_us);
  IRON_REQUIRE(aligned16(embed) && aligned16(angles) && aligned16(x_out) &&
                   (reinterpret_cast<uintptr_t>(exchange) & 255u) == 0 &&
                   (reinterpret_cast<uintptr_t>(attn_workspace) & 255u) == 0 &&
                   (reinterpret_cast<uintptr_t>(keys) & 7u) == 0,
               "%s: embed, angles and x_out must be 16-byte, exchange and workspace 256-byte, keys 8-byte aligned",
               who);
  FusedArgs a;
  a.layers = layers;
  a.n_layers = n_layers;
  a.nsplit = max_len / kDecChunk;
  a.max_len = max_len;
  a.angle_rows = angle_rows;
  a.keys = static_cast<const unsigned long long*>(keys);
  a.n_keys = n_keys;
  a.embed = static_cast<const uint16_t*>(embed);
  a.vocab = vocab;
  a.token = token;
  a.pos = pos;
  a.history = history;
  a.history_cap = history ? history_cap : 0;
  a.angles = angles;
  // the attention workspace as iron_gqa_decode lays it out for 32/8 heads (counters, then partials)
  const long long ctr_bytes = (static_cast<long long>(kNKV) * kCtrStride * 4 + 255) / 256 * 256;
  a.ctr = static_cast<unsigned*>(attn_workspace);
  a.part = reinterpret_cast<float*>(static_cast<char*>(attn_workspace) + ctr_bytes);
  a.head_stride = (static_cast<long long>(a.nsplit) * part_stride<kGQ>() + 63) / 64 * 64;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.eps = eps;
  a.xch = static_cast<unsigned char*>(exchange);
  a.x_out = static_cast<uint16_t*>(x_out);
  a.epoch = epoch;
  a.status = status;
  a.wait_ticks = wait_us * 100u;
  const long long per = kWgQkv + static_cast<long long>(kNKV) * a.nsplit + kWgO + kWgPair + kWgDown;
  const long long grid = kWgSel + per * n_layers;
  IRON_REQUIRE(grid < (1LL << 31), "%s: grid too large", who);
  const dim3 g(static_cast<unsigned>(grid)), blk(256);
  if (flags & IRON_GQA_KV_RESIDENT)
    IRON_LAUNCH(decode_step_kernel<true>, g, blk, 0, static_cast<hipStream_t>(stream), a);
  else
    IRON_LAUNCH(decode_step_kernel<false>, g, blk, 0, static_cast<hipStream_t>(stream), a);
  return check_launch(who);
}
