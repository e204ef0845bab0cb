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
// order, and the shared decode attention body with 64-position chunks), so
// the step's logits are bit-identical to the 82-launch step wherever that
// step's attention takes 64-position chunks too (on long caches it takes 128,
// whose merge sums in another order).
#include "iron_common.hpp"
#include "i4_dot.hpp"
#include "decode_attn.hpp"
#include "exchange.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

constexpr int kE = 2048;                         // hidden size
constexpr int kF = 8192;                         // FFN size
constexpr int kNH = 32, kNKV = 8, kGQ = 4;       // query heads, KV heads, heads per KV head
constexpr int kQKV = (kNH + 2 * kNKV) * kD;      // 3072 q|k|v rows

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

// threadIdx.x as a value the compiler must treat as new at every call: the
// persistent loop then recomputes each thread-dependent address where it is
// used instead of hoisting dozens of them out of the loop and keeping them
// live (which spilled registers).
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Workgroup barrier for LDS only: the weight and cache loads in flight are not waited for.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Waits until pairs [p0, p0 + NP) carry `tag` and leaves their data words in
// dst[0, NP) (LDS). Lanes x = 0-7 of wave 0 first poll pair sent_a x + sent_b
// (relative to p0: the last pair of the last producer on XCD x),
// lane 8 the status word; then every thread loads its share once and re-polls
// only pairs still missing. Whole workgroup (flag: two LDS words); false,
// for every thread alike, when it gave up.
template <int NP>
__device__ bool wait_vector(__amdgpu_buffer_rsrc_t r, unsigned* status, int p0, int sent_a, int sent_b,
                            unsigned tag, unsigned limit, unsigned bit, uint32_t* dst, int* flag) {
  static_assert(NP % 512 == 0, "two pairs per 16-byte load, 256 threads");
  const int tid = opaque_tid();
  if (tid < kWave) {
    const unsigned long long t0 = now_ticks();
    int fail = 0;
    for (;;) {
      const u32x2_v v = ld_pair(r, p0 + sent_a * (tid & 7) + sent_b);
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
  constexpr int NL = NP / 512;         // 16-byte loads per thread
  constexpr int NB = NL < 4 ? NL : 4;  // in flight at once (registers)
  bool ok = true;
#pragma unroll
  for (int i0 = 0; i0 < NL; i0 += NB) {
    u32x4_v v[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) v[i] = ld_pairs2(r, p0 + 2 * (tid + 256 * (i0 + i)));
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if (v[i][1] != tag || v[i][3] != tag) {  // rare: re-poll this pair of pairs
        const unsigned long long t0 = now_ticks();
        while (ok && (v[i][1] != tag || v[i][3] != tag)) {
          if (read_status(status) != 0u || now_ticks() - t0 > limit) ok = false;
          __builtin_amdgcn_s_sleep(1);
          v[i] = ld_pairs2(r, p0 + 2 * (tid + 256 * (i0 + i)));
        }
      }
      *reinterpret_cast<uint2*>(dst + 2 * (tid + 256 * (i0 + i))) = make_uint2(v[i][0], v[i][2]);
    }
  }
  if (!ok) {
    give_up(status, bit);
    flag[1] = 1;
  }
  lds_barrier();
  return flag[1] == 0;
}

// Waits (wave 0, lanes x = 0-7: pair p0 + sa x) until the 8 sentinel pairs
// carry `tag`, without loading the vector: a point in time, not data. Whole
// workgroup; false, for every thread alike, when it gave up.
__device__ bool wait_seen(__amdgpu_buffer_rsrc_t r, unsigned* status, int p0, int sa, unsigned tag, unsigned limit,
                          unsigned bit, int* flag) {
  const int tid = opaque_tid();
  if (tid < kWave) {
    const unsigned long long t0 = now_ticks();
    int fail = 0;
    for (;;) {
      const u32x2_v v = ld_pair(r, p0 + sa * (tid & 7));
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
    if (tid == 0) flag[0] = fail;
  }
  lds_barrier();
  const int f = flag[0];
  if (f == 2 && tid == 0) give_up(status, bit);
  return f == 0;
}

// int4 group-32 GEMV rows held in registers: the codes (16-byte chunks, lane
// l owning groups l + 64 j) and scales of R rows of one or (PAIR) two
// matrices, K = 2048 * GPL.
template <int GPL, int R, bool PAIR>
struct GemvRegs {
  uint4 c[R][GPL];
  uint4 c2[PAIR ? R : 1][GPL];
  uint16_t s[R][GPL];
  uint16_t s2[PAIR ? R : 1][GPL];
};

// Issues the loads of rows row0 .. row0 + R - 1 (streaming: each weight byte is read once per step).
template <int GPL, int R, bool PAIR>
__device__ __forceinline__ void gemv_fetch(GemvRegs<GPL, R, PAIR>& w, const void* codes, const void* scales,
                                           const void* codes2, const void* scales2, int row0) {
  constexpr int G = GPL * kWave;
  constexpr size_t crow = static_cast<size_t>(G) * 16;
  const int lane = opaque_tid() & (kWave - 1);
  // the rows are the wave's (uniform): their bases stay in scalar registers and
  // each lane adds only its own 32-bit offset
  const int row = __builtin_amdgcn_readfirstlane(row0);
  const uint8_t* c = static_cast<const uint8_t*>(codes) + static_cast<size_t>(row) * crow;
  const uint8_t* c2 = static_cast<const uint8_t*>(codes2) + static_cast<size_t>(row) * crow;
  const uint16_t* sc = static_cast<const uint16_t*>(scales) + static_cast<size_t>(row) * G;
  const uint16_t* sc2 = static_cast<const uint16_t*>(scales2) + static_cast<size_t>(row) * G;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
      const unsigned off = static_cast<unsigned>(r * crow) + static_cast<unsigned>(lane + j * kWave) * 16u;
      w.c[r][j] = ld_stream16(c + off);
      if (PAIR) w.c2[r][j] = ld_stream16(c2 + off);
    }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
      const unsigned off = static_cast<unsigned>(r * G + lane + j * kWave);
      w.s[r][j] = sc[off];
      if (PAIR) w.s2[r][j] = sc2[off];
    }
}

// The R row values (bf16 bits) of the rows in w against the K-vector in xs
// (LDS), the arithmetic of gemv_i4_fast<GPL, R, 1, PAIR, NM> for signed
// codes: the same group products, per-row accumulation order over the groups,
// DPP totals, norm scale, SiLU and residual. The groups are taken one at a
// time (each row still sums them in order), which keeps fewer registers live.
template <int GPL, int R, bool PAIR, int NM, bool RESID>
__device__ __forceinline__ void gemv_rows(const GemvRegs<GPL, R, PAIR>& w, const uint32_t* xs, float eps,
                                          const float (&rres)[R], uint16_t (&out)[R]) {
  constexpr int K = GPL * kWave * 32;
  constexpr uint32_t kMagic = 0x43084308u;  // signed codes
  constexpr float kOffset = 136.f;
  const int lane = opaque_tid() & (kWave - 1);
  const uint4* xv = reinterpret_cast<const uint4*>(xs);
  float acc[R], acc2[R], ss = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = acc2[r] = 0.f;
#pragma unroll
  for (int j = 0; j < GPL; ++j) {
    uint4 xr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) xr[q] = xv[(lane + j * kWave) * 4 + q];
    if (NM == NORM_SCALE) {
#pragma unroll
      for (int q = 0; q < 4; ++q) ss = sumsq_chunk(xr[q], ss);
    }
    XGroup xg;
    build_xgroup(xr, xg);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = fmaf(bf16_to_f32(w.s[r][j]), i4_group_total(w.c[r][j], xg, kMagic, kOffset), acc[r]);
      if (PAIR) acc2[r] = fmaf(bf16_to_f32(w.s2[r][j]), i4_group_total(w.c2[r][j], xg, kMagic, kOffset), acc2[r]);
    }
  }
  const float inv = NM == NORM_SCALE ? inv_rms(wave_sum(ss), K, eps) : 1.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float t = wave_sum(acc[r]);
    float t2 = PAIR ? wave_sum(acc2[r]) : 0.f;
    if (NM == NORM_SCALE) {
      t *= inv;
      t2 *= inv;
    }
    float v = PAIR ? silu_f32(t) * t2 : t;
    if (RESID) v += rres[r];
    out[r] = f32_to_bf16(v);
  }
}

// Publishes one bf16 row per wave, rows 4 t + wave: the four meet in LDS and
// go out as two pairs in one 16-byte store at pair p0 + 2 t.
__device__ __forceinline__ void publish_rows4(__amdgpu_buffer_rsrc_t r, int p0, int t, uint16_t v, unsigned tag,
                                              uint16_t* rows_s) {
  const int tid = opaque_tid(), lane = tid & (kWave - 1), wave = tid >> 6;
  if (lane == 0) rows_s[wave] = v;
  lds_barrier();
  if (threadIdx.x == 0) {
    const uint32_t d0 = rows_s[0] | (static_cast<uint32_t>(rows_s[1]) << 16);
    const uint32_t d1 = rows_s[2] | (static_cast<uint32_t>(rows_s[3]) << 16);
    st_pairs2(r, p0 + 2 * t, d0, d1, tag);
  }
}

// The attention's Io inside the step: q (4 heads), k_new and v_new of KV head j
// are waited for in the exchange area and staged in LDS (st[0..255] q,
// [256..319] k, [320..383] v as bf16); the K/V cache rows were loaded ahead
// (kv); the merged output is published as pairs.
struct FusedDecodeIo {
  static constexpr bool kEarly = false;
  static constexpr bool kStaleL1 = true;  // a persistent workgroup may have merged earlier layers' partials
  static constexpr int kMergeChunks = 8;  // the persistent workgroup holds other stages' weights too
  const FusedArgs& fa;
  int qkv_p0, att_p0;
  unsigned tag;
  uint32_t* st;  // 192 words of LDS
  int* flag;
  DecodeKv kv;
  __device__ __forceinline__ bool wait_inputs(int j) const {
    const __amdgpu_buffer_rsrc_t r = xch_rsrc(fa.xch);
    const int tid = opaque_tid();
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
  __device__ __forceinline__ int thread() const { return opaque_tid(); }
  __device__ __forceinline__ void q_pair(int, int t, uint16_t& qx, uint16_t& qp) const {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(st);
    qx = q[t];
    qp = q[t ^ 32];
  }
  __device__ __forceinline__ void new_kv(int, int cq, uint4& kna, uint4& knb, uint4& vna, uint4& vnb) const {
    const uint4* kvn = reinterpret_cast<const uint4*>(st + kGQ * kD / 2);  // k at 16-byte chunk 0.., v at 8..
    kna = kvn[cq];
    knb = kvn[cq + 4];
    vna = kvn[8 + cq];
    vnb = kvn[8 + cq + 4];
  }
  template <bool RES>
  __device__ __forceinline__ DecodeKv kv_rows(const DecodeArgs&, int, int) const {
    return kv;
  }
  __device__ __forceinline__ void store_out(size_t off, uint32_t lo, uint32_t hi) const {
    st_pairs2(xch_rsrc(fa.xch), att_p0 + static_cast<int>(off >> 1), lo, hi, tag);
  }
};

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

// The position of this step (pair 0, published by the select), polled by wave
// 0 and shared through LDS so that every wave takes the same path; -1 when the
// wait gave up.
__device__ int wait_position(const FusedArgs& a, unsigned tag, int* flag) {
  if (threadIdx.x < kWave) {
    const __amdgpu_buffer_rsrc_t r = xch_rsrc(a.xch);
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
    if (threadIdx.x == 0) flag[3] = got ? static_cast<int>(pv[0] & 0x7fffffffu) : -1;
  }
  lds_barrier();
  return flag[3];
}

// The persistent grid: kGrid workgroups, all resident at once (4 per CU), each
// looping over the layers with a fixed share of every stage:
//   workgroups [0, kWgA): wave 4 w + v owns qkv row 4 w + v; the workgroup owns
//     attention chunk w / 8 of KV head w % 8 (w < 8 nsplit) and o rows 4 w + v
//     (w < 512); and two gate/up rows.
//   workgroups [kWgA, kGrid): two gate/up rows per wave and two down rows per
//     wave (K = 8192).
// Weights are loaded into registers well before their stage: the next layer's
// qkv row and K/V rows once the current gate/up stage's input has arrived,
// the o and gate/up rows right after the attention, and on the down
// workgroups the next layer's gate/up and down rows right after the down
// stage. None is held through the attention (its registers), and each is
// issued after a wait, so the next wait for the exchange (loads count in
// order) finds it long landed.
constexpr int kGrid = 1024;
constexpr int kWgA = 768;
constexpr int kWgOrows = 512;  // workgroups with o rows

template <bool RES>
__device__ void loop_a(const FusedArgs& a, unsigned tag, uint32_t* xs, int* flag) {
  __shared__ uint16_t rows_s[4];
  const int w = blockIdx.x, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gw = w * 4 + wave;
  const bool has_att = w < kNKV * a.nsplit, has_o = w < kWgOrows;
  const int j = w % kXcds, s = w / kXcds;  // the attention chunk: all chunks of head j on one XCD
  const __amdgpu_buffer_rsrc_t xr = xch_rsrc(a.xch);
  const float none[1] = {0.f};

  GemvRegs<1, 1, false> wq, wo;
  GemvRegs<1, 2, true> wp;
  DecodeKv kv{};
  if (w == 0) select_role(a, tag);  // first: layer 0 waits for it
  const IronDecodeLayer& L0 = a.layers[0];
  gemv_fetch(wq, L0.qkv_codes, L0.qkv_scales, nullptr, nullptr, gw);
  int pos = 0;
  bool att = false;
  if (has_att) {
    pos = wait_position(a, tag, flag);
    if (pos < 0) return;
    att = s * kDecChunk <= pos && pos < a.max_len && pos < a.angle_rows;
    if (att) kv = load_kv_rows<RES>(opaque_tid(), static_cast<const uint16_t*>(L0.k_cache), static_cast<const uint16_t*>(L0.v_cache),
                                    a.max_len, s * kDecChunk, j);
  }
  for (int l = 0; l < a.n_layers; ++l) {
    const IronDecodeLayer& L = a.layers[l];
    const int base = layer_pairs(l);
    const bool more = l + 1 < a.n_layers;
    // qkv = Wqkv' x * rms(x). Sentinels: layer 0's x comes from the select
    // alone; later ones from the down rows of workgroups kGrid - 8 + x
    // (pairs 4 (w - kWgA) + 3).
    const int sa = l == 0 ? 0 : 4, sb = l == 0 ? kE / 2 - 1 : 4 * (kGrid - kWgA - 8) + 3;
    if (!wait_vector<kE / 2>(xr, a.status, base, sa, sb, tag, a.wait_ticks, kStX, xs, flag)) return;
    // the o row's residual is x itself: taken from the LDS copy now
    const float o_res = bf16_to_f32(reinterpret_cast<const uint16_t*>(xs)[gw & (kE - 1)]);
    {
      uint16_t v[1];
      gemv_rows<1, 1, false, NORM_SCALE, false>(wq, xs, a.eps, none, v);
      publish_rows4(xr, base + kOffQkv, w, v[0], tag, rows_s);
    }
    // attention chunk (a position past the cache publishes zeros from chunk 0;
    // the host never asks for one)
    if (has_att) {
      if (pos >= a.max_len || pos >= a.angle_rows) {
        const int t = opaque_tid();
        if (s == 0 && t < kGQ * kD / 4) st_pairs2(xr, base + kOffAtt + j * (kGQ * kD / 2) + 2 * t, 0u, 0u, tag);
      } else if (att) {
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
        d.trace = nullptr;
        FusedDecodeIo io{a, base + kOffQkv, base + kOffAtt, tag, xs, flag, kv};
        gqa_decode_chunk<kGQ, true, RES, 4>(d, s, j, pos, io);  // always reaches its input wait (flag[2])
        lds_barrier();
        if (flag[2]) return;  // that wait gave up (the status says so)
      }
    }
    // this layer's o and gate/up rows: loaded after the attention (not held
    // through it), ahead of the o stage's wait
    if (has_o) gemv_fetch(wo, L.o_codes, L.o_scales, nullptr, nullptr, gw);
    gemv_fetch(wp, L.gate_codes, L.gate_scales, L.up_codes, L.up_scales, 2 * gw);
    // x1 = x + Wo attn. Sentinels: the last pair of each KV head's merged output.
    if (has_o) {
      if (!wait_vector<kNH * kD / 2>(xr, a.status, base + kOffAtt, kGQ * kD / 2, kGQ * kD / 2 - 1, tag, a.wait_ticks,
                                     kStAtt, xs, flag))
        return;
      const float rres[1] = {o_res};
      uint16_t v[1];
      gemv_rows<1, 1, false, NORM_NONE, true>(wo, xs, a.eps, rres, v);
      publish_rows4(xr, base + kOffX1, w, v[0], tag, rows_s);
    }
    // h = silu(Wg' x1 * rms) * (Wu' x1 * rms). Sentinels: the o rows of
    // workgroups kWgOrows - 8 + x (pairs 2 w + 1). The next layer's qkv row and
    // K/V rows are loaded once x1 is here.
    if (!wait_vector<kE / 2>(xr, a.status, base + kOffX1, 2, 2 * (kWgOrows - 8) + 1, tag, a.wait_ticks, kStX1, xs,
                             flag))
      return;
    if (more) {
      const IronDecodeLayer& N = a.layers[l + 1];
      gemv_fetch(wq, N.qkv_codes, N.qkv_scales, nullptr, nullptr, gw);
      if (att)
        kv = load_kv_rows<RES>(opaque_tid(), static_cast<const uint16_t*>(N.k_cache), static_cast<const uint16_t*>(N.v_cache),
                               a.max_len, s * kDecChunk, j);
    }
    {
      uint16_t v[2];
      gemv_rows<1, 2, true, NORM_SCALE, false>(wp, xs, a.eps, {0.f, 0.f}, v);
      if ((opaque_tid() & (kWave - 1)) == 0) st_pair(xr, base + kOffH + gw, v[0] | (static_cast<uint32_t>(v[1]) << 16), tag);
    }
    lds_barrier();  // every wave is done with xs before the next stage overwrites it
  }
}

template <bool RES>
__device__ void loop_b(const FusedArgs& a, unsigned tag, uint32_t* xs, int* flag) {
  const int w = blockIdx.x, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gw = w * 4 + wave;
  const int drow = 8 * (w - kWgA) + 2 * wave;  // this wave's two down rows
  const __amdgpu_buffer_rsrc_t xr = xch_rsrc(a.xch);
  GemvRegs<1, 2, true> wp;
  GemvRegs<4, 2, false> wd;
  const IronDecodeLayer& L0 = a.layers[0];
  gemv_fetch(wp, L0.gate_codes, L0.gate_scales, L0.up_codes, L0.up_scales, 2 * gw);
  gemv_fetch(wd, L0.down_codes, L0.down_scales, nullptr, nullptr, drow);
  for (int l = 0; l < a.n_layers; ++l) {
    const int base = layer_pairs(l);
    const bool more = l + 1 < a.n_layers;
    if (!wait_vector<kE / 2>(xr, a.status, base + kOffX1, 2, 2 * (kWgOrows - 8) + 1, tag, a.wait_ticks, kStX1, xs,
                             flag))
      return;
    // the down rows' residual is x1 itself: taken from the LDS copy now
    const uint32_t d_res = xs[drow >> 1];
    {
      uint16_t v[2];
      gemv_rows<1, 2, true, NORM_SCALE, false>(wp, xs, a.eps, {0.f, 0.f}, v);
      if ((opaque_tid() & (kWave - 1)) == 0) st_pair(xr, base + kOffH + gw, v[0] | (static_cast<uint32_t>(v[1]) << 16), tag);
    }
    lds_barrier();  // xs is rewritten by the next wait
    // x' = x1 + Wd h. Sentinels: the gate/up rows of workgroups kGrid - 8 + x (pairs 4 w + 3).
    if (!wait_vector<kF / 2>(xr, a.status, base + kOffH, 4, 4 * (kGrid - 8) + 3, tag, a.wait_ticks, kStH, xs, flag))
      return;
    {
      const float rres[2] = {lo_bf16(d_res), hi_bf16(d_res)};
      uint16_t v[2];
      gemv_rows<4, 2, false, NORM_NONE, true>(wd, xs, a.eps, rres, v);
      const uint32_t out = v[0] | (static_cast<uint32_t>(v[1]) << 16);
      if ((opaque_tid() & (kWave - 1)) == 0) {
        st_pair(xr, layer_pairs(l + 1) + (drow >> 1), out, tag);
        if (!more) *reinterpret_cast<uint32_t*>(a.x_out + drow) = out;
      }
    }
    // The next layer's rows, needed from its gate/up stage on (about a layer
    // away): issued once that layer's input x is out (its qkv workgroups have
    // it), so their 28 MB do not queue ahead of that handoff.
    if (more) {
      if (!wait_seen(xr, a.status, layer_pairs(l + 1) + 4 * (kGrid - kWgA - 8) + 3, 4, tag, a.wait_ticks, kStX, flag))
        return;
      const IronDecodeLayer& N = a.layers[l + 1];
      gemv_fetch(wp, N.gate_codes, N.gate_scales, N.up_codes, N.up_scales, 2 * gw);
      gemv_fetch(wd, N.down_codes, N.down_scales, nullptr, nullptr, drow);
    }
    lds_barrier();
  }
}

// RES: the attention's K/V loads are allocating loads (IRON_GQA_KV_RESIDENT).
template <bool RES>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void decode_step_kernel(FusedArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t xs[kF / 2];  // a stage's input vector
  __shared__ int flag[4];
  const unsigned tag = *a.epoch;
  if (blockIdx.x < kWgA)
    loop_a<RES>(a, tag, xs, flag);
  else
    loop_b<RES>(a, tag, xs, flag);
}

}  // namespace
}  // namespace iron

using namespace iron;

#include <mutex>

// The persistent grid needs kGrid workgroups resident at once: at least 256
// CUs holding 4 of them each (occupancy from the compiled kernel's registers
// and LDS). Checked once per device and kernel variant.
static int check_residency(const char* who, bool res) {
  static std::mutex m;
  static int known[64][2];  // 0 unknown, 1 fits, -1 does not
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail_einval("%s: no current device", who);
  std::lock_guard<std::mutex> lock(m);
  int& k = known[dev][res ? 1 : 0];
  if (k == 0) {
    int cus = 0, per_cu = 0;
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const hipError_t e = res ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<true>, 256, 0)
                             : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<false>, 256, 0);
    k = (e == hipSuccess && static_cast<long long>(cus) * per_cu >= kGrid) ? 1 : -1;
    if (k < 0)
      return fail_einval("%s: the device holds %d x %d workgroups of this kernel at once, fewer than its %d", who, cus,
                         per_cu, kGrid);
  }
  return k > 0 ? 0 : fail_einval("%s: the device cannot hold the %d workgroups of this kernel at once", who, kGrid);
}

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
  IRON_REQUIRE(kNKV * a.nsplit <= kWgA, "%s: max_len=%d exceeds %d (one attention chunk per workgroup)", who, max_len,
               kWgA / kNKV * kDecChunk);
  // every workgroup waits for others: the whole grid must be resident at once;
  // the attention merge needs each KV head's chunks on one XCD
  if (int rc = check_residency(who, (flags & IRON_GQA_KV_RESIDENT) != 0)) return rc;
  IRON_REQUIRE(xcd_round_robin(static_cast<hipStream_t>(stream)) == 1,
               "%s: workgroup ids congruent mod 8 do not share an XCD here, or that could not be checked (the first "
               "check per device cannot run under stream capture)", who);
  const dim3 g(kGrid), blk(256);
  if (flags & IRON_GQA_KV_RESIDENT)
    IRON_LAUNCH(decode_step_kernel<true>, g, blk, 0, static_cast<hipStream_t>(stream), a);
  else
    IRON_LAUNCH(decode_step_kernel<false>, g, blk, 0, static_cast<hipStream_t>(stream), a);
  return check_launch(who);
}
